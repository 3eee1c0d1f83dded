// fused_api.hip - the Metal ABI's multi-matrix entry points over one input
// (MTLC/aljabr_metal_matvec_api.h:83-120): matvec pairs and triples sharing
// the activations (the decode step's gate/up and Q/K/V), their batched form,
// and the gated FFN out = W_down . act(W_gate x) * (W_up x). Matrices of one
// type go to one stacked launch (the batch-1 rows kernel, or the matrix-core
// GEMM at batch >= 2); mixed types run one launch each. Activations and
// outputs are device pointers.
#include <cmath>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

bool gguf_type(int t) {
    return t == ALJABR_ROCM_TYPE_F32 || t == ALJABR_ROCM_TYPE_F16 || t == ALJABR_ROCM_TYPE_Q4_0 ||
           t == ALJABR_ROCM_TYPE_Q8_0 || t == ALJABR_ROCM_TYPE_Q4_K || t == ALJABR_ROCM_TYPE_Q6_K;
}

int row_block(int t) {
    return t == ALJABR_ROCM_TYPE_Q4_K || t == ALJABR_ROCM_TYPE_Q6_K ? 256
           : t == ALJABR_ROCM_TYPE_Q4_0 || t == ALJABR_ROCM_TYPE_Q8_0 ? 32
                                                                        : 1;
}

// The gated activation of the Metal FFN kernels (aljabr_metal_kernel_source.m:
// 72-108): SiLU g / (1 + e^-g) with 0 below -20 and g above 20, or for
// kind 2 the tanh GELU with 0 below -10 and g above 10; the product with up,
// 0 when not finite (aljabr_metal_matvec_api.m: activationKind == 2 picks GELU).
__global__ void gated_act_kernel(float *__restrict__ out, const float *__restrict__ gate,
                                 const float *__restrict__ up, long long n, int gelu) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    float act;
    if (gelu) {
        if (g <= -10.0f) act = 0.0f;
        else if (g >= 10.0f) act = g;
        else act = 0.5f * g * (1.0f + tanhf(0.79788456f * (g + 0.044715f * g * g * g)));
    } else {
        if (g <= -20.0f) act = 0.0f;
        else if (g >= 20.0f) act = g;
        else act = g / (1.0f + expf(-g));
    }
    const float y = act * up[i];
    out[i] = isfinite(y) ? y : 0.0f;
}

}  // namespace

// C_i[batch][N_i] = A[batch][K] . B_i^T for i < n: one stacked launch when
// every matrix has the same type and the shape allows, else one per matrix.
int enqueue_matmul_multi(float *const *C, const float *A, const uint8_t *const *B, int K, const int *N,
                         const int *type, int n, int batch) {
    bool same = true;
    for (int i = 1; i < n; ++i) same = same && type[i] == type[0];
    if (same && batch == 1 && type[0] != ALJABR_ROCM_TYPE_F32 && type[0] != ALJABR_ROCM_TYPE_F16) {
        RowsOut outs[3];
        for (int i = 0; i < n; ++i) outs[i] = RowsOut{C[i], B[i], nullptr, N[i]};
        if (enqueue_rows_fused(type[0], outs, n, A, nullptr, 0.0f, K, 0, kRowsStore) == ALJABR_ROCM_OK)
            return ALJABR_ROCM_OK;
    }
    if (same && batch >= 2 && kquant_mfma_type(type[0]) && batch <= kquant_mfma_max_m(type[0])) {
        KqOut outs[3];
        for (int i = 0; i < n; ++i) outs[i] = KqOut{C[i], B[i], N[i]};
        const int rc = enqueue_kquant_mfma_multi(outs, n, A, K, type[0], batch, false);
        if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
    }
    for (int i = 0; i < n; ++i) {
        const int rc = enqueue_matmul_typed(C[i], A, B[i], nullptr, type[i], 0, K, N[i], batch);
        if (rc != ALJABR_ROCM_OK) return rc;
    }
    return ALJABR_ROCM_OK;
}

int enqueue_gated_act(float *out, const float *gate, const float *up, long long n, int kind) {
    if (n <= 0) return ALJABR_ROCM_OK;
    hipLaunchKernelGGL(gated_act_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       current_stream(), out, gate, up, n, kind == 2 ? 1 : 0);
    return ALJABR_ROCM_OK;
}

namespace {

int check_multi(const void *const *C, const void *A, const void *const *B, int K, const int *N, const int *type,
                int n, int batch, const char *what) {
    if (!A) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: null input", what);
    if (K <= 0 || batch <= 0) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: K and batch must be positive", what);
    for (int i = 0; i < n; ++i) {
        if (!C[i] || !B[i] || N[i] <= 0)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: matrix %d needs non-null buffers and N > 0", what, i);
        if (!gguf_type(type[i]))
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "%s: matrix %d has type %d (F32, F16, Q4_0, Q8_0, Q4_K, Q6_K)",
                        what, i, type[i]);
        if (K % row_block(type[i]) != 0)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: K = %d is not a multiple of type %d's block", what, K,
                        type[i]);
    }
    return ALJABR_ROCM_OK;
}

int multi_entry(void *const *C, const void *A, const void *const *B, int K, const int *N, const int *type, int n,
                int batch, const char *what) {
    ALJ_CHECK_READY();
    int rc = check_multi(C, A, B, K, N, type, n, batch, what);
    if (rc != ALJABR_ROCM_OK) return rc;
    float *c[3];
    const uint8_t *b[3];
    for (int i = 0; i < n; ++i) {
        c[i] = static_cast<float *>(C[i]);
        b[i] = static_cast<const uint8_t *>(B[i]);
    }
    rc = enqueue_matmul_multi(c, static_cast<const float *>(A), b, K, N, type, n, batch);
    if (rc != ALJABR_ROCM_OK) return rc;
    return finish_launch(what);
}

int ffn_entry(void *outDown, const void *inA, const void *gateW, const void *upW, const void *downW, int dim,
              int ffnDim, int typeGate, int typeUp, int typeDown, int activationKind, int batch) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(outDown && inA && gateW && upW && downW, "ffn_gated_fused: buffers must be non-null");
    ALJ_REQUIRE(dim > 0 && ffnDim > 0 && batch > 0, "ffn_gated_fused: dim, ffnDim and batch must be positive");
    const void *gu_c[2] = {outDown, outDown};
    const void *gu_b[2] = {gateW, upW};
    const int gu_n[2] = {ffnDim, ffnDim}, gu_t[2] = {typeGate, typeUp};
    int rc = check_multi(gu_c, inA, gu_b, dim, gu_n, gu_t, 2, batch, "ffn_gated_fused");
    if (rc != ALJABR_ROCM_OK) return rc;
    const void *d_c[1] = {outDown};
    const void *d_b[1] = {downW};
    const int d_n[1] = {dim}, d_t[1] = {typeDown};
    rc = check_multi(d_c, inA, d_b, ffnDim, d_n, d_t, 1, batch, "ffn_gated_fused");
    if (rc != ALJABR_ROCM_OK) return rc;
    const long long hn = static_cast<long long>(batch) * ffnDim;
    const long long hs = (hn + 63) & ~63LL;        // 256-byte aligned pieces
    float *scratch = static_cast<float *>(stream_scratch(static_cast<size_t>(3 * hs) * sizeof(float)));
    if (!scratch) return ALJABR_ROCM_ERR_BUFFER;
    float *gate = scratch, *up = scratch + hs, *h = scratch + 2 * hs;
    float *gu[2] = {gate, up};
    const uint8_t *gw[2] = {static_cast<const uint8_t *>(gateW), static_cast<const uint8_t *>(upW)};
    rc = enqueue_matmul_multi(gu, static_cast<const float *>(inA), gw, dim, gu_n, gu_t, 2, batch);
    if (rc != ALJABR_ROCM_OK) return rc;
    enqueue_gated_act(h, gate, up, hn, activationKind);
    float *od[1] = {static_cast<float *>(outDown)};
    const uint8_t *dw[1] = {static_cast<const uint8_t *>(downW)};
    rc = enqueue_matmul_multi(od, h, dw, ffnDim, d_n, d_t, 1, batch);
    if (rc != ALJABR_ROCM_OK) return rc;
    return finish_launch("ffn_gated_fused");
}

}  // namespace
}  // namespace aljabr

using namespace aljabr;

extern "C" {

int aljabr_rocm_matvec_tb_pair(void *C0, void *C1, const void *A, const void *B0, const void *B1, int K, int N0,
                               int N1, int type0, int type1) {
    void *C[2] = {C0, C1};
    const void *B[2] = {B0, B1};
    const int N[2] = {N0, N1}, T[2] = {type0, type1};
    return multi_entry(C, A, B, K, N, T, 2, 1, "matvec_tb_pair");
}

int aljabr_rocm_matvec_tb_triple(void *C0, void *C1, void *C2, const void *A, const void *B0, const void *B1,
                                 const void *B2, int K, int N0, int N1, int N2, int type0, int type1, int type2) {
    void *C[3] = {C0, C1, C2};
    const void *B[3] = {B0, B1, B2};
    const int N[3] = {N0, N1, N2}, T[3] = {type0, type1, type2};
    return multi_entry(C, A, B, K, N, T, 3, 1, "matvec_tb_triple");
}

int aljabr_rocm_matvec_tb_triple_batch(void *C0, void *C1, void *C2, const void *A, const void *B0, const void *B1,
                                       const void *B2, int K, int N0, int N1, int N2, int type0, int type1, int type2,
                                       int batchSize) {
    void *C[3] = {C0, C1, C2};
    const void *B[3] = {B0, B1, B2};
    const int N[3] = {N0, N1, N2}, T[3] = {type0, type1, type2};
    return multi_entry(C, A, B, K, N, T, 3, batchSize, "matvec_tb_triple_batch");
}

int aljabr_rocm_ffn_gated_fused(void *outDown, const void *inA, const void *gateW, const void *upW, const void *downW,
                                int dim, int ffnDim, int typeGate, int typeUp, int typeDown, int activationKind) {
    return ffn_entry(outDown, inA, gateW, upW, downW, dim, ffnDim, typeGate, typeUp, typeDown, activationKind, 1);
}

int aljabr_rocm_ffn_gated_fused_batch(void *outDown, const void *inA, const void *gateW, const void *upW,
                                      const void *downW, int dim, int ffnDim, int typeGate, int typeUp, int typeDown,
                                      int activationKind, int batchSize) {
    return ffn_entry(outDown, inA, gateW, upW, downW, dim, ffnDim, typeGate, typeUp, typeDown, activationKind,
                     batchSize);
}

}  // extern "C"
