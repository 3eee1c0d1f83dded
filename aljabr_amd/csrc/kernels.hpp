// kernels.hpp - stream-ordered enqueue functions shared between the C-ABI
// entry points and the decode-step driver. None of them synchronises; each
// returns an ALJABR_ROCM_* status.
#pragma once

#include <cstdint>

namespace aljabr {

struct AttnParams {
    float *out;             // fp32, same layout as q
    const float *q;         // fp32; [B][Hq][Sq][D] unless the strides below say otherwise
    const void *k, *v;      // [B][Hkv][cap][D] (or paged, below), fp16 or fp32
    const float *mask;      // [Sq][Sk] additive, or null
    const int *kv_len;      // per-batch visible key count (device), or null for Sk
    int B, Hq, Hkv, Sq, Sk, D, cap;
    float scale;
    int causal;
    int kv_f16;
    // Paged caches [phys][Hkv][block_size][D]: key j of sequence b is row
    // j % block_size of block block_table[b * max_blocks + j / block_size].
    const int *block_table; // null: contiguous caches
    int block_size, max_blocks;
    // Key range rule of the paged Metal ABI (MTLC/aljabr_metal_attention.m:146-160,
    // :192-200) instead of CpuBackend's: query position query_start + qi
    // (bottom-right when causal without a window and query_start == 0),
    // optional sliding window.
    int paged_bounds, query_start, window;
    float soft_cap;         // > 0: score = soft_cap * tanh(score / soft_cap)
    float norm_eps;         // output = O / (L + norm_eps)
    long long q_sb, q_sh, q_sq;   // element strides of q and out (0: [B][Hq][Sq][D])
    float *scratch;         // split partials: caller-owned (graph-safe) when it holds attention_scratch_bytes(),
    size_t scratch_bytes;   // else (null or too small) the stream's scratch
    int scratch_only;       // never use the stream's scratch: fewer splits when the partials would not fit
    // With Sq == 1 and out as [B][Hq*D]: the output also as the NF4 GEMM's
    // fp16 A image over K = Hq*D (rows past B untouched); enqueue_attention
    // returns UNSUPPORTED, before any launch, where its kernels cannot write it.
    uint16_t *xpack;
};

int enqueue_attention(const AttnParams &p);
// Upper bound of the split-partial bytes enqueue_attention needs for B
// sequences of Hq heads, Sq query rows, head size D and `keys` cached keys.
size_t attention_scratch_bytes(int B, int Hq, int Sq, int D, int keys);

// Small-M GEMMs use the matrix-core kernels unless ALJABR_ROCM_MFMA=0.
bool mfma_enabled();
// C[M][N] = A[M][K] . W[N][K]^T for any M (slices or MFMA chosen inside).
// `part`/`part_floats`: a caller-owned buffer for the matrix-core kernels'
// K-slice partials (nf4_mfma_scratch_floats / kquant_mfma_scratch_floats of
// the pass); when null or too small they take the stream's scratch.
int enqueue_matmul_nf4(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs, int M,
                       float *part = nullptr, size_t part_floats = 0);
int enqueue_matmul_gguf(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M,
                        float *part = nullptr, size_t part_floats = 0);
int enqueue_matmul_f32(float *C, const float *A, const float *W, int K, int N, int M);
// Any weight type of the library (NF4 with its absmax and block size, GGUF
// F32/F16/Q4_0/Q8_0/Q4_K/Q6_K).
int enqueue_matmul_typed(float *C, const float *A, const void *W, const float *absmax, int type, int bs, int K, int N,
                         int M, float *part = nullptr, size_t part_floats = 0);
// GGUF Q4_K / Q6_K rows (K % 256 == 0, A and W 16-byte aligned), any M.
int enqueue_matmul_kquant(float *C, const float *A, const uint8_t *W, int K, int N, int type, int M,
                          float *part = nullptr, size_t part_floats = 0);
// GGUF block-format (Q4_K, Q6_K, Q4_0, Q8_0) small-M GEMM on MFMA
// (2 <= M <= kquant_mfma_max_m(type): 32 for the K-quants, 8 for Q4_0 and
// Q8_0; K % 512 == 0, A and W 16-byte aligned; ALJABR_ROCM_ERR_UNSUPPORTED
// otherwise, nothing enqueued).
bool kquant_mfma_type(int type);
int kquant_mfma_max_m(int type);
int enqueue_kquant_mfma(float *C, const float *A, const uint8_t *W, int K, int N, int type, int M,
                        float *part = nullptr, size_t part_floats = 0);
// Floats of `part` one enqueue_kquant_mfma_multi launch of M tokens over N
// stacked rows and K needs (0: a single K slice).
size_t kquant_mfma_scratch_floats(int M, int N, int K);
// The same over up to three matrices of one type and K stacked in one launch
// (all but the last with a multiple of 32 rows); outs[i].y is [M][outs[i].n].
// With `accumulate` the products are added to the outputs as they are.
struct KqOut {
    float *y;
    const uint8_t *w;
    int n;
};
// With several 512-element K slices the partial sums go to `part` (at least
// (K / 512) * M * (stacked rows) floats) or, when that is null or too small,
// to the stream's scratch; `accumulate` adds the product into the outputs.
// `xpacked`: A's fp16 image (nf4_xpack_bytes layout) for the Q4_K
// register-resident kernel where it takes the shape (ignored otherwise).
struct SliceTail;
int enqueue_kquant_mfma_multi(const KqOut *outs, int nseg, const float *A, int K, int type, int M, bool accumulate,
                              float *part = nullptr, size_t part_floats = 0, const SliceTail *tail = nullptr,
                              const uint16_t *xpacked = nullptr);
// The K slices' products only (K >= 1024), into part[slice][m][col0 + stacked
// row] with row stride ld (part holds slices * M * ld floats, col0 % 32 == 0):
// launches of different types stacked in one buffer, then one slice tail.
int enqueue_kquant_mfma_parts(const KqOut *outs, int nseg, const float *A, int K, int type, int M, float *part,
                              size_t part_floats, int ld, int col0);
// The same for two types in one launch (Q4_K matrices, then Q6_K ones, all
// over the same x): part[slice][m][stacked row of both] with row stride the
// rows of both, or UNSUPPORTED (other types, or more workgroups than CUs).
int enqueue_kquant_mfma_parts2(const KqOut *outs0, int nseg0, int type0, const KqOut *outs1, int nseg1, int type1,
                               const float *A, int K, int M, float *part, size_t part_floats);
// ys[s] (+)= the K slices' partial sums part[slice][m][stacked row] of
// segment s (stacked rows [ends[s-1], ends[s])), added in slice order.
int enqueue_slice_sum(float *const *ys, const int *ends, int nseg, int M, int N, const float *part, int slices,
                      bool add);
// y = cap * tanh(y / cap) elementwise.
int enqueue_softcap(float *y, long long n, float cap);
// K-split tile kernels for M <= 2 (ALJABR_ROCM_ERR_UNSUPPORTED when the shape
// or alignment does not fit them; nothing is enqueued then).
int enqueue_nf4_tile(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M);
int enqueue_gguf_tile(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M);
// Batch-1 NF4 kernel: T rows per workgroup, one wave per 2048-element K
// chunk (K <= 16384, K % 2048 == 0, block size >= 32).
int enqueue_nf4_rows(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift);
// Batch-1 NF4/Q4_0/Q8_0/Q4_K/Q6_K kernel, a 256-entry pair table for NF4 and
// Q4_0 codes (K % 2048 == 0, K <= 16384; NF4 block size >= 32, 16-byte
// aligned codes; Q4_0/Q8_0 rows 4-byte aligned, K-quant rows 16-byte
// aligned). `type` is an ALJABR_ROCM_TYPE_* id.
// C[M][N] = A[M][K] . W^T for M = 2..4 NF4 tokens on the batch-1 rows kernel
// (fp32); ALJABR_ROCM_ERR_UNSUPPORTED (nothing launched) outside its limits.
int enqueue_rows_nf4_mt(float *C, const float *A, const uint8_t *W, const float *absmax, int K, int N, int bs_shift,
                        int M);
int enqueue_rows(float *C, const float *A, const uint8_t *W, const float *absmax, int K, int N, int type,
                 int bs_shift);
// One weight matrix of a fused batch-1 NF4 launch: y[0..n) = W[n][K] . x'.
struct RowsOut {
    float *y;
    const uint8_t *w;
    const float *absmax;
    int n;
};
// The sequence and caches of a Q/K/V launch that rotates and appends (one
// sequence: pos[0]; caches of one layer [n_kv][cap][head_dim] fp16).
struct RowsRope {
    const int *pos;
    uint16_t *kc, *vc;
    int cap, head_dim;
    float base;
    const float2 *cs;   // [cap][head_dim/2] cos/sin table (enqueue_rope_table), or null
    int n_kv;           // KV heads in the caches ([n_kv][cap][head_dim] each)
};
constexpr int kRowsStore = 0;    // y = W x'
constexpr int kRowsAdd = 1;      // y += W x' (residual; no norm prologue)
constexpr int kRowsSwiGLU = 2;   // outs = {gate, up}: outs[0].y = silu(Wg x') * (Wu x')
constexpr int kRowsRopeKV = 3;   // outs = {q, k, v}: q rotated into outs[0].y; k rotated and v appended to the caches
constexpr int kRowsGeGLU = 4;    // as kRowsSwiGLU with the Metal FFN's tanh GELU: gelu(Wg x') * (Wu x')
// Batch-1 NF4 matvec of up to three matrices sharing K and the activations
// (stacked rows, one launch). x' = RMSNorm(x) with weight norm_w when norm_w
// is non-null (over the K elements), else x. Same shape limits as
// enqueue_rows, even row counts; ALJABR_ROCM_ERR_UNSUPPORTED (nothing
// enqueued) outside them.
int enqueue_nf4_rows_fused(const RowsOut *outs, int nseg, const float *x, const float *norm_w, float eps, int K,
                           int bs_shift, int epilogue, const RowsRope *rope = nullptr);
// The same for one weight type shared by the segments: NF4, Q4_0, Q8_0, Q4_K
// or Q6_K (absmax and bs_shift for NF4 only).
int enqueue_rows_fused(int type, const RowsOut *outs, int nseg, const float *x, const float *norm_w, float eps, int K,
                       int bs_shift, int epilogue, const RowsRope *rope = nullptr);
// RMSNorm + Q and K in type01 + V in type2 in one launch (Q4_K beside Q6_K),
// with RoPE and the cache append (kRowsRopeKV) or stored (kRowsStore), or
// UNSUPPORTED.
int enqueue_rows_mixed(int type01, int type2, const RowsOut *outs, const float *x, const float *norm_w, float eps,
                       int K, int epilogue, const RowsRope *rope = nullptr);
// What the second kernel of a split-K GEMM does with the slice sums besides
// (or instead of) writing them: the decode step's next element-wise launch,
// applied to the stacked rows of the GEMM (slice_tails.hip).
constexpr int kTailSwiGLU = 1;        // rows [0, n) gate, [n, 2n) up: out[m][i] = silu(gate) * up
constexpr int kTailRopeAppend = 2;    // rows q (nh heads), k, v (nkv heads): out = rotated q; k (rotated) and v
                                      // appended as fp16 at row pos[m] of caches [M][nkv][cap][head_dim]
constexpr int kTailResidualNorm = 3;  // out[m] += sums (residual); xn[m] = RMSNorm(out[m]) * norm_w
// kTailResidualScale: y += the slice sums, xn = y * norm_w (no row scale),
// and per (row, column block) sums of squares of y to ssq[M][kSsqParts];
// a later tail with `ssq` set applies RMSNorm's row scale 1/sqrt(mean + eps)
// to its slice sums (W.(x*s*w) = s*(W.(x*w)) for a per-row scale s), which
// spreads the residual step over many workgroups instead of one per row.
constexpr int kTailResidualScale = 4;
constexpr int kSsqParts = 8;
struct SliceTail {
    int kind;
    float *out;
    int n;
    uint16_t *kc, *vc;
    const int *pos;
    int nh, nkv, head_dim, cap;
    float base;
    const float2 *cs;
    float *xn;
    const float *norm_w;
    float eps;
    // Row scale of a preceding kTailResidualScale (SwiGLU and RoPE tails):
    // ssq[M][kSsqParts] over rows of norm_n elements, or null for none.
    float *ssq;
    int norm_n;
    // Also the output as the NF4 matrix-core GEMM's fp16 A image (the layout
    // nf4_xpack_kernel writes; rows >= M left as they are), when the next
    // GEMM consumes it: the SwiGLU and residual tails; null for none.
    uint16_t *xpack;
};
int enqueue_slice_tail(const SliceTail &t, const float *part, int slices, int M, int N);
// NF4 small-M GEMM on MFMA (M >= 2 in passes of 64 tokens, K % 256 == 0,
// block size 64), deterministic: C = A . W^T, or with `add` C += A . W^T (a
// residual). K % 1024 == 0 runs the register-resident kernel (activations
// rounded to fp16, levels exact: about 2e-4 relative per row), other K the
// fp32-accurate LDS-staged one. When K is split over workgroups the partial
// sums (and the fp16 activation image) go to `part`
// (nf4_mfma_scratch_floats(M, N, K) floats) or, when that is null or too
// small, to the stream's scratch, and a second kernel adds the slices in
// order.
int enqueue_nf4_mfma(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M, bool add = false, float *part = nullptr, size_t part_floats = 0);
// The same over up to three matrices of one K stacked in one launch (all but
// the last with a multiple of 32 rows); outs[i].y is [M][outs[i].n].
// With `tail` (M <= 64) the outputs are not written: the slice sums go to
// the tail kernel instead (outs[].y unused).
// `xpacked`: A already as the GEMM's fp16 A image (a tail's xpack, M <= 64),
// or null.
int enqueue_nf4_mfma_multi(const RowsOut *outs, int nseg, const float *A, int K, int bs_shift, int M, bool add,
                           float *part = nullptr, size_t part_floats = 0, const SliceTail *tail = nullptr,
                           const uint16_t *xpacked = nullptr);
// Bytes of the fp16 A image for M <= 64 tokens over K (K % 64 == 0).
size_t nf4_xpack_bytes(int M, int K);
// GGUF Q4_0 / Q8_0 GEMM pass of M <= 16 tokens with the activations held in
// registers (K % 2048 == 0, A 16-byte aligned; up to three stacked matrices
// of one type, all but the last a multiple of 16 rows; fp32-accurate,
// deterministic). With several K slices or a tail the partial sums go to
// `part` (K / 2048 * M * (stacked rows) floats suffice) or the stream's
// scratch. ALJABR_ROCM_ERR_UNSUPPORTED when the shape does not fit.
int gguf_gemm_pass(const RowsOut *outs, int nseg, const float *A, int K, int type, int M, bool add, float *part,
                   size_t part_floats, const SliceTail *tail);
// Q4_K GEMM pass of M <= 64 tokens with the activations held in registers
// as fp16 (rounded once: an A image built first, or `xpacked`; K % 4096 ==
// 0, A 16-byte aligned, up to three stacked matrices, all but the last a
// multiple of 16 rows; deterministic). Partials and the image go to `part`
// (q4k_gemm_scratch_floats(M, N, K) floats suffice) or the stream's scratch.
// ALJABR_ROCM_ERR_UNSUPPORTED when the shape does not fit.
int q4k_gemm_pass(const RowsOut *outs, int nseg, const float *A, int K, int M, bool add, float *part,
                  size_t part_floats, const SliceTail *tail, const uint16_t *xpacked);
size_t q4k_gemm_scratch_floats(int M, int N, int K);
// Floats of `part` enqueue_nf4_mfma_multi needs for M tokens over N stacked
// rows and K (every pass, with or without a tail, xpacked null).
size_t nf4_mfma_scratch_floats(int M, int N, int K);
// The plan enqueue_nf4_mfma_multi uses for N stacked rows over K on `cus`
// CUs and passes of M tokens (row tiles per wave, sub-slices per K slice),
// and one pass of at most 64 tokens under an explicit plan (segments as enqueue_nf4_mfma_multi,
// already validated).
void nf4_mfma_plan(int N, int K, int M, int cus, int &nt, int &q);
int nf4_mfma_pass_planned(const RowsOut *outs, int nseg, const float *A, int K, int M, bool add, float *part,
                          size_t part_floats, int nt, int q, const SliceTail *tail = nullptr);
// fp16-weight small-M GEMM on MFMA (2 <= M <= 32, K in {512, 1024, 2048,
// 4096}, W and A 16-byte aligned); deterministic (no atomics).
int enqueue_f16_mfma(float *C, const float *A, const uint16_t *W, int K, int N, int M);
// Persistent double-buffered batch-1 kernels (K <= 16384).
int enqueue_gguf_stream(float *C, const float *A, const uint8_t *B, int K, int N, int type);
// Small-M (M <= 8) wavefront-reduction kernels.
int enqueue_nf4_small(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs, int M);
int enqueue_gguf_small(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M);

int enqueue_rmsnorm(float *out, const float *x, const float *w, int rows, int len, float eps);
int enqueue_rope(float *x, const int *pos, int rows, int n_heads, int head_dim, float base);
int enqueue_swiglu(float *dst, const float *gate, const float *up, long long n);
int enqueue_add(float *a, const float *b, long long n);
// out = act(gate) * up of the Metal FFN kernels (kind 2: tanh GELU, else
// SiLU, with their cut-offs; a non-finite product becomes 0).
int enqueue_gated_act(float *out, const float *gate, const float *up, long long n, int kind);
// C_i[batch][N_i] = A[batch][K] . B_i^T for i < n (n <= 3) over any GGUF
// weight types: matrices of one type share one stacked launch where the
// shape allows (the batch-1 rows kernel, the matrix-core GEMM at batch >= 2),
// else one launch each.
int enqueue_matmul_multi(float *const *C, const float *A, const uint8_t *const *B, int K, const int *N,
                         const int *type, int n, int batch);
// Argmax of each row (ties to the lowest index, NaN never taken, 0 for a row
// with nothing above -inf). With `part` of at least argmax_part_bytes(rows,
// cols) bytes (8-byte aligned) it runs as chunk maxima plus a final pass (no
// workgroup reads a whole wide row), else one workgroup per row.
int enqueue_argmax(int *out, const float *x, int rows, int cols, void *part = nullptr, size_t part_bytes = 0);
size_t argmax_part_bytes(int rows, int cols);
int enqueue_embed(float *x, const float *embed, const int *tokens, int batch, int dim, int vocab);
// x[b] = row tokens[b] of a [vocab][dim] table of type F32, F16, Q4_0, Q8_0,
// Q4_K or Q6_K, decoded bit-exactly (dim a multiple of the type's block).
int enqueue_embed_typed(float *x, const void *table, int type, const int *tokens, int batch, int dim, int vocab);
int enqueue_kv_append(uint16_t *cache, const float *src, const int *pos, int batch, int n_kv, int head_dim, int cap);
// RoPE on q [batch][nh][D] in place and on k, then k and v [batch][nkv][D]
// appended as fp16 at row pos[b] of caches [batch][nkv][cap][D] (D/2 <= 1024).
// `cs` is a table from enqueue_rope_table for (cap, head_dim, base), or null.
int enqueue_rope_append(float *q, const float *k, const float *v, uint16_t *kc, uint16_t *vc, const int *pos, int batch,
                        int nh, int nkv, int head_dim, int cap, float base, const float2 *cs);
// cs[p][i] = (cos, sin) of RoPE pair i at position p, p < cap, i < head_dim/2,
// the values the RoPE kernels would compute for that position.
int enqueue_rope_table(float2 *cs, int cap, int head_dim, float base);

}  // namespace aljabr
