// step_api.hip - the Metal ABI's registered whole-step decode and its fused
// layer entry points (MTLC/aljabr_metal_matvec_api.h:161-282): a KV cache and
// per-layer weights registered once (init_kv_cache, register_norm_buffer,
// register_rope_freqs, register_decode_layer, register_output,
// register_token_embd), then one call per generated token (decode_step,
// decode_step_token) that runs every layer and the logits on the device, and
// the per-layer calls the prefill path uses (wo_ffn_fused*, the batched
// wo_ffn_fused_layer_batch).
//
// The registry is process-wide, as the reference's is: one model at a time,
// calls serialised by a mutex, each call finished on its stream before it
// returns (the reference waits for its command buffer). Data pointers may be
// host or device memory: device pointers are used in place, host weights are
// uploaded once (cached by address), host norms and inputs are copied in and
// outputs copied back. The KV caches are fp32 and position-major, as the
// reference lays them out ([max_seq][stride] per layer), so sync_kv_cache is
// a plain copy; attention reads them as a paged cache of one-row blocks.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kMaxStepLayers = 256;
constexpr int kThreads = 256;

// ---- device kernels ---------------------------------------------------------

__device__ __forceinline__ float step_block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) t += red[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
    return 1.0f / static_cast<float>(sqrt(static_cast<double>(ss / static_cast<float>(n) + eps)));
}

__global__ void set_i32_kernel(int *p, int v) { *p = v; }

// Per-head preparation of one token's Q/K/V (MTLC/aljabr_metal_matvec_api.m:
// 3648-3790): block b < nh is Q head b (head norm, RoPE, in place); the next
// nkv blocks are K heads (head norm, RoPE, stored to the cache row `pos`);
// the last nkv are V heads (unit norm, stored), read from the raw K
// projection when the layer has no V projection. The RoPE angle is
// pos * base^(-2i/D) / ff with ff the layer's positive divisor for pair i
// (1 when absent or not positive).
struct HeadPrep {
    float *q;
    const float *k, *v;          // v null: K as V
    float *kc, *vc;              // row pos of this layer's caches, or null when nothing is stored
    const float *qn_w, *kn_w;    // head-norm weights [D], null: no norm
    const float *freqs;
    int nfreqs;
    int nh, nkv, hd;
    int pos, unit_v;
    float base, eps;
};

__global__ __launch_bounds__(kThreads) void head_prep_kernel(HeadPrep a) {
    __shared__ float red[kThreads / 64];
    const int b = blockIdx.x;
    const int kind = b < a.nh ? 0 : b < a.nh + a.nkv ? 1 : 2;
    const int head = kind == 0 ? b : kind == 1 ? b - a.nh : b - a.nh - a.nkv;
    const int hd = a.hd, half = hd >> 1;
    const float *src = (kind == 0 ? a.q : kind == 1 ? a.k : (a.v ? a.v : a.k)) + static_cast<long long>(head) * hd;
    const float *w = kind == 0 ? a.qn_w : kind == 1 ? a.kn_w : nullptr;
    const bool norm = kind == 2 ? a.unit_v != 0 : w != nullptr;
    float inv = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < hd; i += blockDim.x) ss = fmaf(src[i], src[i], ss);
        inv = inv_rms(step_block_sum(ss, red), hd, a.eps);
    }
    float *dst = kind == 0 ? a.q + static_cast<long long>(head) * hd
                           : (kind == 1 ? a.kc : a.vc) + static_cast<long long>(head) * hd;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float x0 = src[i], x1 = src[i + half];
        if (norm) {
            x0 *= inv;
            x1 *= inv;
            if (w) {
                x0 *= w[i];
                x1 *= w[i + half];
            }
        }
        if (kind != 2) {
            float c, s;
            const float ff = (a.freqs && i < a.nfreqs) ? a.freqs[i] : 1.0f;
            if (ff > 0.0f && ff != 1.0f) {
                const float exponent = -2.0f * static_cast<float>(i) / static_cast<float>(hd);
                const float inv_freq = static_cast<float>(pow(static_cast<double>(a.base), static_cast<double>(exponent)));
                const float theta = static_cast<float>(a.pos) * inv_freq / ff;
                c = static_cast<float>(cos(static_cast<double>(theta)));
                s = static_cast<float>(sin(static_cast<double>(theta)));
            } else {
                rope_cos_sin(a.pos, i, hd, a.base, c, s);
            }
            rope_apply(x0, x1, c, s);
        }
        dst[i] = x0;
        dst[i + half] = x1;
    }
}

// One row per workgroup (MTLC/aljabr_metal_kernel_source.m:905-964):
// xb = post_w ? rmsnorm(xb) * post_w : xb; x += xb; xb = rmsnorm(x) * ffn_w.
__global__ __launch_bounds__(1024) void post_attn_ffn_norm_kernel(float *__restrict__ xb, float *__restrict__ x,
                                                                  const float *__restrict__ post_w,
                                                                  const float *__restrict__ ffn_w, int n, float eps) {
    __shared__ float red[1024 / 64];
    float *br = xb + static_cast<long long>(blockIdx.x) * n;
    float *xr = x + static_cast<long long>(blockIdx.x) * n;
    float inv = 1.0f;
    if (post_w) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(br[i], br[i], ss);
        inv = inv_rms(step_block_sum(ss, red), n, eps);
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float b = post_w ? (br[i] * inv) * post_w[i] : br[i];
        const float v = xr[i] + b;
        xr[i] = v;
        ss = fmaf(v, v, ss);
    }
    const float inv2 = inv_rms(step_block_sum(ss, red), n, eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) br[i] = (xr[i] * inv2) * ffn_w[i];
}

// One row per workgroup (MTLC/aljabr_metal_kernel_source.m:966-1011):
// xb = post_w ? rmsnorm(xb) * post_w : xb; x = (x + xb) * scale, the scale
// applied only when positive and not 1.
__global__ __launch_bounds__(1024) void post_ffn_scale_kernel(const float *__restrict__ xb, float *__restrict__ x,
                                                              const float *__restrict__ post_w, int n, float eps,
                                                              float scale) {
    __shared__ float red[1024 / 64];
    const float *br = xb + static_cast<long long>(blockIdx.x) * n;
    float *xr = x + static_cast<long long>(blockIdx.x) * n;
    float inv = 1.0f;
    if (post_w) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(br[i], br[i], ss);
        inv = inv_rms(step_block_sum(ss, red), n, eps);
    }
    const bool apply = scale > 0.0f && scale != 1.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float b = post_w ? (br[i] * inv) * post_w[i] : br[i];
        const float v = xr[i] + b;
        xr[i] = apply ? v * scale : v;
    }
}

// x[r] *= s for every element of `rows` rows (the embedding scale).
__global__ void scale_kernel(float *__restrict__ x, long long n, float s) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) x[i] *= s;
}

// ---- host side --------------------------------------------------------------

bool weight_type_ok(int t) {
    return t == ALJABR_ROCM_TYPE_F32 || t == ALJABR_ROCM_TYPE_F16 || t == ALJABR_ROCM_TYPE_Q4_0 ||
           t == ALJABR_ROCM_TYPE_Q8_0 || t == ALJABR_ROCM_TYPE_Q4_K || t == ALJABR_ROCM_TYPE_Q6_K;
}

int type_block(int t) {
    return t == ALJABR_ROCM_TYPE_Q4_K || t == ALJABR_ROCM_TYPE_Q6_K   ? 256
           : t == ALJABR_ROCM_TYPE_Q4_0 || t == ALJABR_ROCM_TYPE_Q8_0 ? 32
                                                                        : 1;
}

// Bytes of an [n][k] matrix of type t (k a whole number of blocks).
size_t matrix_bytes(int t, long long n, long long k) {
    switch (t) {
    case ALJABR_ROCM_TYPE_F32: return static_cast<size_t>(n * k * 4);
    case ALJABR_ROCM_TYPE_F16: return static_cast<size_t>(n * k * 2);
    case ALJABR_ROCM_TYPE_Q4_0: return static_cast<size_t>(n * (k / 32) * 18);
    case ALJABR_ROCM_TYPE_Q8_0: return static_cast<size_t>(n * (k / 32) * 34);
    case ALJABR_ROCM_TYPE_Q4_K: return static_cast<size_t>(n * (k / 256) * 144);
    default: return static_cast<size_t>(n * (k / 256) * 210);
    }
}

bool is_device_ptr(const void *p) {
    if (!p) return false;
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    bool ensure(size_t bytes) {
        if (bytes <= cap && p) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = (bytes + 4095) & ~size_t(4095);
        if (hipMalloc(&p, want) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            return false;
        }
        cap = want;
        return true;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
    float *f() const { return static_cast<float *>(p); }
};

struct Mat {
    const uint8_t *w = nullptr;  // device data, null: absent
    int type = 0;
};

// A host weight buffer uploaded once: keyed by its address, byte count and
// type, so a different model at a reused address with another size or type
// never reads the old copy.
struct UploadKey {
    const void *p;
    size_t bytes;
    int type;
    bool operator==(const UploadKey &o) const { return p == o.p && bytes == o.bytes && type == o.type; }
};
struct UploadKeyHash {
    size_t operator()(const UploadKey &k) const {
        return std::hash<const void *>()(k.p) ^ (std::hash<size_t>()(k.bytes) * 31u) ^ (static_cast<size_t>(k.type) << 7);
    }
};

struct Layer {
    bool set = false;
    std::vector<UploadKey> uploads;     // host weights this registration uploaded
    int kv_layer = 0, owner = 0;
    Mat q, k, v, o, gate, up, down;
    int n0 = 0, n1 = 0, n2 = 0, wo_k = 0, wo_n = 0, ffn = 0, nh = 0, nkv = 0, hd = 0, stride = 0;
    float freq_base = 10000.0f;
    int is_swa = 0;
    float out_scale = 1.0f, attn_scale = 0.0f;
    int post_attn = 0, post_ffn = 0, q_norm = 0, k_norm = 0, unit_v = 0;
    DevBuf freqs;
    int nfreqs = 0;
};

struct NormSlot {
    const float *p = nullptr;    // device view
    size_t bytes = 0;
    DevBuf owned;                // the copy of a host buffer
};

struct Upload {
    DevBuf buf;
    int owners = 0;              // registrations (layers, output, embedding) holding it
};

struct State {
    std::mutex mu;
    int kv_layers = 0, kv_max_seq = 0;
    std::vector<int> kv_stride;
    std::vector<DevBuf> kv_k, kv_v;
    DevBuf block_ids;            // identity block table [max_seq]
    NormSlot norm[6];
    Layer layer[kMaxStepLayers];
    int num_layers = 0;
    bool geometry_ready = false;
    int dim = 0, max_q = 0, max_kv = 0, max_att = 0, max_ffn = 0, max_hd = 0;
    Mat out_w;
    const float *out_norm = nullptr;
    DevBuf out_norm_owned;
    int out_k = 0, out_n = 0;
    float cap = 0.0f;
    Mat embd;
    int embd_dim = 0, embd_vocab = 0;
    float embd_scale = 1.0f;
    int activation = 2;
    // activations
    DevBuf x, xb, att, q, k, v, gate, up, hb, logits, ints, staging, next_norm;
    std::vector<UploadKey> out_uploads, embd_uploads;
    std::unordered_map<UploadKey, Upload, UploadKeyHash> uploads;

    void release_all() {
        for (auto &b : kv_k) b.release();
        for (auto &b : kv_v) b.release();
        kv_k.clear();
        kv_v.clear();
        kv_stride.clear();
        kv_layers = kv_max_seq = 0;
        block_ids.release();
        for (auto &s : norm) {
            s.owned.release();
            s.p = nullptr;
            s.bytes = 0;
        }
        for (auto &l : layer) {
            l.freqs.release();
            l = Layer();
        }
        num_layers = 0;
        geometry_ready = false;
        out_w = Mat();
        out_norm = nullptr;
        out_norm_owned.release();
        out_k = out_n = 0;
        cap = 0.0f;
        embd = Mat();
        embd_dim = embd_vocab = 0;
        embd_scale = 1.0f;
        activation = 2;
        for (DevBuf *b : {&x, &xb, &att, &q, &k, &v, &gate, &up, &hb, &logits, &ints, &staging, &next_norm})
            b->release();
        for (auto &u : uploads) u.second.buf.release();
        uploads.clear();
        out_uploads.clear();
        embd_uploads.clear();
    }
};

State &state() {
    static State s;
    return s;
}

// Device view of weights: device memory in place, host memory uploaded once
// per (address, bytes, type). With `owner` the upload is held by that
// registration (listed there, released by drop_uploads when it is
// registered again); without, it stays cached for later calls.
int device_weights(State &st, const void *p, size_t bytes, int type, const uint8_t **out,
                   std::vector<UploadKey> *owner = nullptr) {
    if (!p) {
        *out = nullptr;
        return ALJABR_ROCM_OK;
    }
    if (is_device_ptr(p)) {
        *out = static_cast<const uint8_t *>(p);
        return ALJABR_ROCM_OK;
    }
    const UploadKey key{p, bytes, type};
    Upload &u = st.uploads[key];
    if (!u.buf.p) {
        if (!u.buf.ensure(bytes)) {
            st.uploads.erase(key);
            return fail(ALJABR_ROCM_ERR_BUFFER, "weight upload: cannot allocate %zu bytes", bytes);
        }
        const hipError_t e = hipMemcpy(u.buf.p, p, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            st.uploads.erase(key);
            return fail(ALJABR_ROCM_ERR_DEVICE, "weight upload: %s", hipGetErrorString(e));
        }
    }
    if (owner) {
        ++u.owners;
        owner->push_back(key);
    }
    *out = static_cast<const uint8_t *>(u.buf.p);
    return ALJABR_ROCM_OK;
}

// A registration is replaced: its uploads lose an owner, and those no other
// registration holds are freed (the host buffers may hold other weights now).
void drop_uploads(State &st, std::vector<UploadKey> &keys) {
    for (const UploadKey &k : keys) {
        auto it = st.uploads.find(k);
        if (it != st.uploads.end() && --it->second.owners <= 0) {
            it->second.buf.release();
            st.uploads.erase(it);
        }
    }
    keys.clear();
}

// Copy `bytes` from host or device memory into device memory (stream order).
int copy_in(void *dst, const void *src, size_t bytes, hipStream_t s) {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, is_device_ptr(src) ? hipMemcpyDeviceToDevice
                                                                           : hipMemcpyHostToDevice, s);
    return e == hipSuccess ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_DEVICE, "copy in: %s", hipGetErrorString(e));
}

int copy_out(void *dst, const void *src, size_t bytes, hipStream_t s) {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, is_device_ptr(dst) ? hipMemcpyDeviceToDevice
                                                                           : hipMemcpyDeviceToHost, s);
    return e == hipSuccess ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_DEVICE, "copy out: %s", hipGetErrorString(e));
}

int sync(hipStream_t s, const char *what) {
    const hipError_t e = hipStreamSynchronize(s);
    return e == hipSuccess ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

// A call that fails part-way may leave work queued: wait for it, so that the
// next call (maybe on another stream) finds the shared buffers idle.
int drained(int rc) {
    if (rc < 0 && aljabr_rocm_is_initialized()) {
        (void)hipStreamSynchronize(current_stream());
        (void)hipGetLastError();
    }
    return rc;
}

int launch_ok(const char *what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

// y[rows][n] = x[rows][k] . W^T
int matmul(float *y, const float *x, const Mat &m, int k, int n, int rows) {
    return enqueue_matmul_typed(y, x, m.w, nullptr, m.type, 0, k, n, rows);
}

// Registered-matrix checks: type, and K a whole number of the type's blocks.
int check_mat(const void *w, int type, int n, int k, const char *name) {
    if (!w) return ALJABR_ROCM_OK;
    if (!weight_type_ok(type)) return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "%s: weight type %d is not supported", name, type);
    if (n <= 0 || k <= 0 || k % type_block(type) != 0)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: [%d x %d] does not fit type %d blocks", name, n, k, type);
    return ALJABR_ROCM_OK;
}

// Resolve KV owners and size the activation buffers for `rows` token rows
// (MTLC/aljabr_metal_matvec_api.m:3222-3266).
int prepare(State &st, int rows) {
    if (!st.geometry_ready) {
        const Layer &l0 = st.layer[0];
        st.dim = l0.wo_n;
        st.max_q = st.max_kv = st.max_att = st.max_ffn = st.max_hd = 0;
        for (int l = 0; l < st.num_layers; ++l) {
            Layer &c = st.layer[l];
            st.max_q = std::max(st.max_q, c.n0);
            st.max_kv = std::max(st.max_kv, std::max(c.n1, c.n2));
            st.max_att = std::max(st.max_att, c.wo_k);
            st.max_ffn = std::max(st.max_ffn, c.ffn);
            st.max_hd = std::max(st.max_hd, c.hd);
            int owner = c.kv_layer, hops = 0;
            while (owner >= 0 && owner < st.num_layers && hops++ < st.num_layers) {
                const Layer &cand = st.layer[owner];
                if (cand.k.w || cand.kv_layer == owner) break;
                owner = cand.kv_layer;
            }
            c.owner = owner;
        }
        st.geometry_ready = true;
    }
    const size_t r = static_cast<size_t>(std::max(rows, 1));
    const size_t wide = static_cast<size_t>(std::max(st.dim, st.max_att));
    bool ok = st.x.ensure(r * st.dim * 4) && st.xb.ensure(r * wide * 4) && st.att.ensure(r * wide * 4) &&
              st.q.ensure(r * (st.max_q + 4) * 4) && st.k.ensure(r * (st.max_kv + 4) * 4) &&
              st.v.ensure(r * (st.max_kv + 4) * 4) && st.gate.ensure(r * st.max_ffn * 4) &&
              st.up.ensure(r * st.max_ffn * 4) && st.hb.ensure(r * st.max_ffn * 4) &&
              st.logits.ensure(static_cast<size_t>(std::max(st.out_n, 1)) * 4) && st.ints.ensure(256);
    return ok ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_BUFFER, "decode step: cannot allocate activations");
}

// Norm slot row `l` of a [layers][n] slot, or null when the slot is absent;
// an error when it is present but too short.
int slot_row(const State &st, int slot, int l, int n, const float **out) {
    const NormSlot &s = st.norm[slot];
    *out = nullptr;
    if (!s.p) return ALJABR_ROCM_OK;
    if ((static_cast<size_t>(l) + 1) * n * 4 > s.bytes)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "norm slot %d holds %zu bytes, layer %d needs %zu", slot, s.bytes, l,
                    (static_cast<size_t>(l) + 1) * n * 4);
    *out = s.p + static_cast<size_t>(l) * n;
    return ALJABR_ROCM_OK;
}

// Attention sub-layer input to residual, then the FFN, for `rows` rows held
// in st.x (residual) and st.att (attention output), layer `l`'s registered
// weights: MTLC/aljabr_metal_matvec_api.m:3866-3989 (one row) and :4202-4350
// (rows). `fast` allows the fused batch-1 rows launches.
struct FfnLayer {
    Mat o, gate, up, down;
    int wo_k, dim, ffn;
    const float *post_attn, *ffn_norm, *post_ffn;
    float out_scale;
};

int wo_ffn(State &st, const FfnLayer &f, int rows, float eps, int act) {
    float *x = st.x.f(), *xb = st.xb.f(), *att = st.att.f(), *hb = st.hb.f();
    int rc;
    bool ffn_in_ready = false;   // xb = ffn_norm(x)
    bool hb_ready = false;
    bool attn_added = false;
    if (rows == 1 && !f.post_attn) {
        const RowsOut o{x, f.o.w, nullptr, f.dim};
        rc = enqueue_rows_fused(f.o.type, &o, 1, att, nullptr, eps, f.wo_k, 0, kRowsAdd);
        if (rc == ALJABR_ROCM_OK) attn_added = true;
        else if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
    }
    if (!attn_added) {
        if ((rc = matmul(xb, att, f.o, f.wo_k, f.dim, rows))) return rc;
        hipLaunchKernelGGL(post_attn_ffn_norm_kernel, dim3(rows), dim3(1024), 0, current_stream(), xb, x, f.post_attn,
                           f.ffn_norm, f.dim, eps);
        ffn_in_ready = true;
    } else if (f.gate.type == f.up.type) {
        const RowsOut gu[2] = {{hb, f.gate.w, nullptr, f.ffn}, {hb, f.up.w, nullptr, f.ffn}};
        rc = enqueue_rows_fused(f.gate.type, gu, 2, x, f.ffn_norm, eps, f.dim, 0, act == 2 ? kRowsGeGLU : kRowsSwiGLU);
        if (rc == ALJABR_ROCM_OK) hb_ready = true;
        else if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
    }
    if (!hb_ready) {
        if (!ffn_in_ready && (rc = enqueue_rmsnorm(xb, x, f.ffn_norm, rows, f.dim, eps))) return rc;
        float *gu_y[2] = {st.gate.f(), st.up.f()};
        const uint8_t *gu_w[2] = {f.gate.w, f.up.w};
        const int gu_n[2] = {f.ffn, f.ffn}, gu_t[2] = {f.gate.type, f.up.type};
        if ((rc = enqueue_matmul_multi(gu_y, xb, gu_w, f.dim, gu_n, gu_t, 2, rows))) return rc;
        if ((rc = enqueue_gated_act(hb, st.gate.f(), st.up.f(), static_cast<long long>(rows) * f.ffn, act))) return rc;
    }
    const bool plain_add = !f.post_ffn && !(f.out_scale > 0.0f && f.out_scale != 1.0f);
    if (rows == 1 && plain_add) {
        const RowsOut d{x, f.down.w, nullptr, f.dim};
        rc = enqueue_rows_fused(f.down.type, &d, 1, hb, nullptr, eps, f.ffn, 0, kRowsAdd);
        if (rc == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
        if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
    }
    if ((rc = matmul(xb, hb, f.down, f.ffn, f.dim, rows))) return rc;
    hipLaunchKernelGGL(post_ffn_scale_kernel, dim3(rows), dim3(1024), 0, current_stream(), xb, x, f.post_ffn, f.dim,
                       eps, f.out_scale);
    return ALJABR_ROCM_OK;
}

// Logits of st.x (one row) into st.logits, softcap applied; the greedy token
// to st.ints[0].
int logits_step(State &st, const Mat &w, const float *norm_w, int k, int n, float cap, float eps) {
    float *lg = st.logits.f();
    int rc;
    const RowsOut o{lg, w.w, nullptr, n};
    rc = enqueue_rows_fused(w.type, &o, 1, st.x.f(), norm_w, eps, k, 0, kRowsStore);
    if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
        if ((rc = enqueue_rmsnorm(st.xb.f(), st.x.f(), norm_w, 1, k, eps))) return rc;
        rc = matmul(lg, st.xb.f(), w, k, n, 1);
    }
    if (rc) return rc;
    if (cap > 0.0f && (rc = enqueue_softcap(lg, n, cap))) return rc;
    return enqueue_argmax(static_cast<int *>(st.ints.p), lg, 1, n);
}

// The whole step for one token (MTLC/aljabr_metal_matvec_api.m:3574-4083).
int decode_step_locked(State &st, int pos, int window, float eps, const float *x_in, int token, float *logits_out) {
    ALJ_CHECK_READY();
    if (st.num_layers == 0) return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "decode_step: no decode layer is registered");
    for (int l = 0; l < st.num_layers; ++l)
        if (!st.layer[l].set) return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "decode_step: layer %d is not registered", l);
    if (!st.norm[3].p || !st.norm[1].p)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "decode_step: the attention (slot 3) and FFN (slot 1) norms are required");
    if (st.kv_layers < st.num_layers) return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "decode_step: KV cache covers %d of %d layers",
                                                  st.kv_layers, st.num_layers);
    if (pos < 0 || pos >= st.kv_max_seq)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: position %d outside the cache (%d)", pos, st.kv_max_seq);
    int rc = prepare(st, 1);
    if (rc) return rc;
    hipStream_t s = current_stream();
    const int dim = st.dim;
    float *x = st.x.f();
    if (token >= 0) {
        if (!st.embd.w || st.embd_dim != dim || token >= st.embd_vocab)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step_token: token %d without a matching embedding", token);
        hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, s, static_cast<int *>(st.ints.p) + 1, token);
        if ((rc = enqueue_embed_typed(x, st.embd.w, st.embd.type, static_cast<int *>(st.ints.p) + 1, 1, dim,
                                      st.embd_vocab)))
            return rc;
        if (st.embd_scale != 1.0f)
            hipLaunchKernelGGL(scale_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, x, static_cast<long long>(dim),
                               st.embd_scale);
    } else {
        if (!x_in) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: x_in is null");
        if ((rc = copy_in(x, x_in, static_cast<size_t>(dim) * 4, s))) return rc;
    }
    int *kv_len = static_cast<int *>(st.ints.p) + 2;
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, s, kv_len, pos + 1);
    for (int l = 0; l < st.num_layers; ++l) {
        const Layer &c = st.layer[l];
        if (c.wo_n != dim) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: layer %d width %d != %d", l, c.wo_n, dim);
        const float *attn_norm, *ffn_norm, *post_attn, *post_ffn, *qn = nullptr, *kn = nullptr;
        if ((rc = slot_row(st, 3, l, dim, &attn_norm)) || (rc = slot_row(st, 1, l, dim, &ffn_norm)) ||
            (rc = slot_row(st, 0, l, dim, &post_attn)) || (rc = slot_row(st, 2, l, dim, &post_ffn)))
            return rc;
        if (c.q_norm && (rc = slot_row(st, 4, l, st.max_hd, &qn))) return rc;
        if (c.k_norm && c.k.w && (rc = slot_row(st, 5, l, st.max_hd, &kn))) return rc;
        if (!c.post_attn) post_attn = nullptr;
        if (!c.post_ffn) post_ffn = nullptr;
        // Q, K, V from the attention-normed residual: the matrices of one
        // type share a batch-1 rows launch with the RMSNorm as its prologue;
        // shapes that launch cannot take go through the normed copy in xb.
        float *q = st.q.f(), *k = st.k.f(), *v = st.v.f();
        {
            const Mat mats[3] = {c.q, c.k, c.v};
            float *const ys[3] = {q, k, v};
            const int ns[3] = {c.n0, c.n1, c.n2};
            bool done[3] = {false, c.k.w == nullptr, c.v.w == nullptr};
            bool xb_ready = false;
            if (c.k.w && c.v.w && c.q.type == c.k.type && c.v.type != c.q.type) {
                // Q4_K q and k beside a Q6_K v: one launch of two row formats.
                const RowsOut outs[3] = {{q, c.q.w, nullptr, c.n0}, {k, c.k.w, nullptr, c.n1}, {v, c.v.w, nullptr, c.n2}};
                rc = enqueue_rows_mixed(c.q.type, c.v.type, outs, x, attn_norm, eps, dim, kRowsStore);
                if (rc == ALJABR_ROCM_OK) done[0] = done[1] = done[2] = true;
                else if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
            }
            for (int i = 0; i < 3; ++i) {
                if (done[i]) continue;
                RowsOut outs[3];
                int idx[3], n = 0;
                for (int j = i; j < 3; ++j)
                    if (!done[j] && mats[j].type == mats[i].type) {
                        outs[n] = RowsOut{ys[j], mats[j].w, nullptr, ns[j]};
                        idx[n++] = j;
                    }
                rc = enqueue_rows_fused(mats[i].type, outs, n, x, attn_norm, eps, dim, 0, kRowsStore);
                if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                    if (!xb_ready) {
                        if ((rc = enqueue_rmsnorm(st.xb.f(), x, attn_norm, 1, dim, eps))) return rc;
                        xb_ready = true;
                    }
                    for (int j = 0; j < n; ++j)
                        if ((rc = matmul(ys[idx[j]], st.xb.f(), mats[idx[j]], dim, ns[idx[j]], 1))) return rc;
                } else if (rc != ALJABR_ROCM_OK) {
                    return rc;
                }
                for (int j = 0; j < n; ++j) done[idx[j]] = true;
            }
        }
        if (c.k.w && !c.v.w && (c.n1 <= 0 || c.n1 != c.n2))
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: layer %d K-as-V needs n1 == n2", l);
        // KV owner and geometry (MTLC/aljabr_metal_matvec_api.m:3798-3831).
        const int owner = c.owner;
        if (owner < 0 || owner >= st.num_layers || owner >= st.kv_layers || !st.layer[owner].k.w)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: layer %d has no KV owner with a K projection", l);
        const Layer &oc = st.layer[owner];
        if (oc.hd != c.hd || oc.nkv != c.nkv || st.kv_stride[owner] < c.nkv * c.hd)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: layer %d KV geometry differs from its owner %d", l,
                        owner);
        if (st.kv_stride[owner] != c.nkv * c.hd)
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED,
                        "decode_step: KV stride %d of layer %d is not n_kv_heads * head_dim = %d", st.kv_stride[owner],
                        owner, c.nkv * c.hd);
        if (c.hd < 2 || (c.hd & 1)) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: odd head_dim %d", c.hd);
        if (c.k.w && st.kv_stride[l] < c.nkv * c.hd)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: layer %d cache stride %d < n_kv_heads * head_dim",
                        l, st.kv_stride[l]);
        HeadPrep hp{};
        hp.q = q;
        hp.k = k;
        hp.v = c.v.w ? v : nullptr;
        const bool store = c.k.w != nullptr;
        if (store) {
            hp.kc = st.kv_k[l].f() + static_cast<long long>(pos) * st.kv_stride[l];
            hp.vc = st.kv_v[l].f() + static_cast<long long>(pos) * st.kv_stride[l];
        }
        hp.qn_w = qn;
        hp.kn_w = kn;
        hp.freqs = c.nfreqs ? c.freqs.f() : nullptr;
        hp.nfreqs = c.nfreqs;
        hp.nh = c.nh;
        hp.nkv = c.nkv;
        hp.hd = c.hd;
        hp.pos = pos;
        hp.unit_v = c.unit_v;
        hp.base = c.freq_base;
        hp.eps = eps;
        hipLaunchKernelGGL(head_prep_kernel, dim3(c.nh + (store ? 2 * c.nkv : 0)), dim3(kThreads), 0, s, hp);
        // Attention over the owner's cache, keys [start, pos].
        float scale = c.attn_scale;
        if (scale <= 0.0f)
            scale = (c.q_norm || c.k_norm) ? 1.0f : static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.hd)));
        AttnParams p{};
        p.out = st.att.f();
        p.q = q;
        p.k = st.kv_k[owner].p;
        p.v = st.kv_v[owner].p;
        p.kv_len = kv_len;
        p.B = 1;
        p.Hq = c.nh;
        p.Hkv = oc.nkv;
        p.Sq = 1;
        p.Sk = pos + 1;
        p.D = c.hd;
        p.cap = 0;
        p.scale = scale;
        p.causal = 1;
        p.kv_f16 = 0;
        p.block_table = static_cast<const int *>(st.block_ids.p);
        p.block_size = 1;
        p.max_blocks = pos + 1;
        p.paged_bounds = 1;
        p.query_start = pos;
        p.window = c.is_swa && window > 0 ? window : 0;
        p.soft_cap = 0.0f;
        p.norm_eps = 1e-9f;
        if ((rc = enqueue_attention(p))) return rc;
        FfnLayer f{c.o, c.gate, c.up, c.down, c.wo_k, dim, c.ffn, post_attn, ffn_norm, post_ffn, c.out_scale};
        if ((rc = wo_ffn(st, f, 1, eps, st.activation))) return rc;
    }
    int best = 0;
    const bool have_out = st.out_w.w && st.out_norm && st.out_n > 0;
    if (have_out) {
        if (st.out_k != dim) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step: output K %d != %d", st.out_k, dim);
        if ((rc = logits_step(st, st.out_w, st.out_norm, st.out_k, st.out_n, st.cap, eps))) return rc;
        if (logits_out && (rc = copy_out(logits_out, st.logits.p, static_cast<size_t>(st.out_n) * 4, s))) return rc;
        if (hipMemcpyAsync(&best, st.ints.p, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess)
            return fail(ALJABR_ROCM_ERR_DEVICE, "decode_step: %s", hipGetErrorString(hipGetLastError()));
    }
    if ((rc = launch_ok("decode_step"))) return rc;
    if ((rc = sync(s, "decode_step"))) return rc;
    return best;
}

// Inputs of the ad-hoc fused calls: device views of host or device vectors,
// staged after `used` bytes of st.staging.
const float *view_in(State &st, const void *p, size_t bytes, size_t &used, hipStream_t s, int &rc) {
    if (!p) return nullptr;
    if (is_device_ptr(p)) return static_cast<const float *>(p);
    char *dst = static_cast<char *>(st.staging.p) + used;
    used += (bytes + 255) & ~size_t(255);
    const hipError_t e = hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) rc = fail(ALJABR_ROCM_ERR_DEVICE, "copy in: %s", hipGetErrorString(e));
    return reinterpret_cast<const float *>(dst);
}

struct AdHoc {
    float *x;
    const float *attn_full;
    const void *wO;
    int typeWO, wO_K, wO_N;
    const float *postAttnW;
    int hasPostAttnNorm;
    const float *ffnNormW, *postFfnW;
    int hasPostFfnNorm;
    float eps, outScale;
    const void *gateW, *upW, *downW;
    int typeGate, typeUp, typeDown, ffnDim, activationKind;
};

// wO + norms + FFN + residual for the caller's pointers
// (MTLC/aljabr_metal_matvec_api.m:2198-2658): x and attn_full are copied in,
// the weights resolved; the caller then adds its tail (next layer's Q/K/V or
// the logits) and copies out.
int adhoc_layer(State &st, const AdHoc &a, hipStream_t s, size_t &used) {
    if (!a.x || !a.attn_full || !a.wO || !a.ffnNormW || !a.gateW || !a.upW || !a.downW)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "wo_ffn_fused: x, attn_full, weights and the FFN norm are required");
    if (a.wO_K <= 0 || a.wO_N <= 0 || a.ffnDim <= 0)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "wo_ffn_fused: dimensions must be positive");
    int rc;
    if ((rc = check_mat(a.wO, a.typeWO, a.wO_N, a.wO_K, "wO")) || (rc = check_mat(a.gateW, a.typeGate, a.ffnDim, a.wO_N, "gate")) ||
        (rc = check_mat(a.upW, a.typeUp, a.ffnDim, a.wO_N, "up")) ||
        (rc = check_mat(a.downW, a.typeDown, a.wO_N, a.ffnDim, "down")))
        return rc;
    Mat o, g, u, d;
    o.type = a.typeWO;
    g.type = a.typeGate;
    u.type = a.typeUp;
    d.type = a.typeDown;
    if ((rc = device_weights(st, a.wO, matrix_bytes(a.typeWO, a.wO_N, a.wO_K), a.typeWO, &o.w)) ||
        (rc = device_weights(st, a.gateW, matrix_bytes(a.typeGate, a.ffnDim, a.wO_N), a.typeGate, &g.w)) ||
        (rc = device_weights(st, a.upW, matrix_bytes(a.typeUp, a.ffnDim, a.wO_N), a.typeUp, &u.w)) ||
        (rc = device_weights(st, a.downW, matrix_bytes(a.typeDown, a.wO_N, a.ffnDim), a.typeDown, &d.w)))
        return rc;
    const size_t db = static_cast<size_t>(a.wO_N) * 4;
    // x, attn_full and up to four norm vectors staged.
    if (!st.staging.ensure(6 * ((db + static_cast<size_t>(a.wO_K) * 4 + 255) & ~size_t(255)) + 4096))
        return fail(ALJABR_ROCM_ERR_BUFFER, "wo_ffn_fused: cannot allocate staging");
    if ((rc = copy_in(st.x.p, a.x, db, s)) || (rc = copy_in(st.att.p, a.attn_full, static_cast<size_t>(a.wO_K) * 4, s)))
        return rc;
    rc = ALJABR_ROCM_OK;
    const float *ffn_norm = view_in(st, a.ffnNormW, db, used, s, rc);
    const float *post_attn = a.hasPostAttnNorm ? view_in(st, a.postAttnW, db, used, s, rc) : nullptr;
    const float *post_ffn = a.hasPostFfnNorm ? view_in(st, a.postFfnW, db, used, s, rc) : nullptr;
    if (rc) return rc;
    FfnLayer f{o, g, u, d, a.wO_K, a.wO_N, a.ffnDim, post_attn, ffn_norm, post_ffn, a.outScale};
    return wo_ffn(st, f, 1, a.eps, a.activationKind);
}

// Size the shared activations for an ad-hoc call of width dim, attention
// width k, FFN ffn and (optionally) a vocab.
int adhoc_prepare(State &st, int dim, int k, int ffn, int qn, int vocab) {
    const size_t wide = static_cast<size_t>(std::max(dim, k));
    const bool ok = st.x.ensure(static_cast<size_t>(dim) * 4) && st.xb.ensure(wide * 4) && st.att.ensure(wide * 4) &&
                    st.gate.ensure(static_cast<size_t>(ffn) * 4) && st.up.ensure(static_cast<size_t>(ffn) * 4) &&
                    st.hb.ensure(static_cast<size_t>(ffn) * 4) && st.q.ensure((static_cast<size_t>(qn) + 4) * 4) &&
                    st.k.ensure((static_cast<size_t>(qn) + 4) * 4) && st.v.ensure((static_cast<size_t>(qn) + 4) * 4) &&
                    st.logits.ensure(static_cast<size_t>(std::max(vocab, 1)) * 4) && st.ints.ensure(256);
    return ok ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_BUFFER, "wo_ffn_fused: cannot allocate activations");
}

}  // namespace

void step_state_release() {
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    st.release_all();
}

}  // namespace aljabr

using namespace aljabr;

extern "C" {

int aljabr_rocm_init_kv_cache(int nLayers, int maxSeq, const int *layerStrides) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        ALJ_REQUIRE(nLayers > 0 && nLayers <= kMaxStepLayers && maxSeq > 0 && layerStrides,
                    "init_kv_cache: 1 <= nLayers <= %d, maxSeq > 0 and the strides are required", kMaxStepLayers);
        for (int i = 0; i < nLayers; ++i)
            ALJ_REQUIRE(layerStrides[i] > 0, "init_kv_cache: stride of layer %d must be positive", i);
        for (auto &b : st.kv_k) b.release();
        for (auto &b : st.kv_v) b.release();
        st.kv_k.assign(nLayers, DevBuf());
        st.kv_v.assign(nLayers, DevBuf());
        st.kv_stride.assign(layerStrides, layerStrides + nLayers);
        st.kv_layers = nLayers;
        st.kv_max_seq = maxSeq;
        hipStream_t s = current_stream();
        for (int i = 0; i < nLayers; ++i) {
            const size_t bytes = static_cast<size_t>(maxSeq) * layerStrides[i] * 4;
            if (!st.kv_k[i].ensure(bytes) || !st.kv_v[i].ensure(bytes)) {
                st.kv_layers = 0;
                return fail(ALJABR_ROCM_ERR_BUFFER, "init_kv_cache: cannot allocate layer %d (%zu bytes)", i, bytes);
            }
            if (hipMemsetAsync(st.kv_k[i].p, 0, bytes, s) != hipSuccess || hipMemsetAsync(st.kv_v[i].p, 0, bytes, s) != hipSuccess)
                return fail(ALJABR_ROCM_ERR_DEVICE, "init_kv_cache: clear failed");
        }
        if (!st.block_ids.ensure(static_cast<size_t>(maxSeq) * 4))
            return fail(ALJABR_ROCM_ERR_BUFFER, "init_kv_cache: cannot allocate the block table");
        std::vector<int> ids(maxSeq);
        for (int i = 0; i < maxSeq; ++i) ids[i] = i;
        if (hipMemcpy(st.block_ids.p, ids.data(), ids.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return fail(ALJABR_ROCM_ERR_DEVICE, "init_kv_cache: block table upload failed");
        return sync(s, "init_kv_cache");
    }());
}

int aljabr_rocm_sync_kv_cache(int layer, int seqLen, const float *kData, const float *vData) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        ALJ_REQUIRE(layer >= 0 && layer < st.kv_layers && seqLen > 0 && seqLen <= st.kv_max_seq,
                    "sync_kv_cache: layer %d / seqLen %d outside the cache (%d layers, %d positions)", layer, seqLen,
                    st.kv_layers, st.kv_max_seq);
        hipStream_t s = current_stream();
        const size_t bytes = static_cast<size_t>(seqLen) * st.kv_stride[layer] * 4;
        int rc;
        if (kData && (rc = copy_in(st.kv_k[layer].p, kData, bytes, s))) return rc;
        if (vData && (rc = copy_in(st.kv_v[layer].p, vData, bytes, s))) return rc;
        return sync(s, "sync_kv_cache");
    }());
}

int aljabr_rocm_register_norm_buffer(int slot, const void *ptr, size_t bytes) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    ALJ_REQUIRE(slot >= 0 && slot < 6 && ptr && bytes > 0, "register_norm_buffer: slot 0..5, a buffer and its size");
    NormSlot &n = st.norm[slot];
    if (is_device_ptr(ptr)) {
        n.owned.release();
        n.p = static_cast<const float *>(ptr);
    } else {
        if (!n.owned.ensure(bytes)) return fail(ALJABR_ROCM_ERR_BUFFER, "register_norm_buffer: cannot allocate");
        if (hipMemcpy(n.owned.p, ptr, bytes, hipMemcpyHostToDevice) != hipSuccess)
            return fail(ALJABR_ROCM_ERR_DEVICE, "register_norm_buffer: upload failed");
        n.p = n.owned.f();
    }
    n.bytes = bytes;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_register_rope_freqs(int layer, const float *freqData, int freqLen) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        ALJ_REQUIRE(layer >= 0 && layer < kMaxStepLayers && freqData && freqLen > 0,
                    "register_rope_freqs: layer 0..%d, data and a positive length", kMaxStepLayers - 1);
        Layer &l = st.layer[layer];
        if (!l.freqs.ensure(static_cast<size_t>(freqLen) * 4))
            return fail(ALJABR_ROCM_ERR_BUFFER, "register_rope_freqs: cannot allocate");
        hipStream_t s = current_stream();
        int rc = copy_in(l.freqs.p, freqData, static_cast<size_t>(freqLen) * 4, s);
        if (rc) return rc;
        l.nfreqs = freqLen;
        return sync(s, "register_rope_freqs");
    }());
}

int aljabr_rocm_register_decode_layer(int layer, int kvLayerIndex, const void *wQ, const void *wK, const void *wV,
                                      const void *wO, const void *gate, const void *up, const void *down, int typeQ,
                                      int typeK, int typeV, int typeWO, int typeGate, int typeUp, int typeDown, int n0,
                                      int n1, int n2, int wO_K, int wO_N, int ffnDim, int nH, int nKVH, int headDim,
                                      int stride, float freqBase, int isSwa, float outScale, float attnScale,
                                      int hasPostAttnNorm, int hasPostFfnNorm, int hasQNorm, int hasKNorm,
                                      int hasUnitVNorm) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    ALJ_REQUIRE(layer >= 0 && layer < kMaxStepLayers, "register_decode_layer: layer %d outside 0..%d", layer,
                kMaxStepLayers - 1);
    ALJ_REQUIRE(kvLayerIndex >= 0 && kvLayerIndex <= layer, "register_decode_layer: kvLayerIndex %d must be in 0..%d",
                kvLayerIndex, layer);
    ALJ_REQUIRE(wQ && wO && up && down && gate, "register_decode_layer: wQ, wO, gate, up and down are required");
    ALJ_REQUIRE(nH > 0 && nKVH > 0 && headDim > 0 && n0 == nH * headDim && wO_K == n0 && wO_N > 0 && ffnDim > 0,
                "register_decode_layer: n0 = wO_K = nH * headDim and positive sizes");
    ALJ_REQUIRE(!wK || n1 == nKVH * headDim, "register_decode_layer: n1 must be nKVH * headDim");
    ALJ_REQUIRE(!wV || n2 == nKVH * headDim, "register_decode_layer: n2 must be nKVH * headDim");
    int rc;
    if ((rc = check_mat(wQ, typeQ, n0, wO_N, "wQ")) || (rc = check_mat(wK, typeK, n1, wO_N, "wK")) ||
        (rc = check_mat(wV, typeV, n2, wO_N, "wV")) || (rc = check_mat(wO, typeWO, wO_N, wO_K, "wO")) ||
        (rc = check_mat(gate, typeGate, ffnDim, wO_N, "gate")) || (rc = check_mat(up, typeUp, ffnDim, wO_N, "up")) ||
        (rc = check_mat(down, typeDown, wO_N, ffnDim, "down")))
        return rc;
    Layer &c = st.layer[layer];
    // Registering again replaces the layer: its old uploads are dropped first
    // (a failed registration leaves the layer unregistered).
    c.set = false;
    drop_uploads(st, c.uploads);
    st.geometry_ready = false;
    Mat mq, mk, mv, mo, mg, mu, md;
    mq.type = typeQ; mk.type = typeK; mv.type = typeV; mo.type = typeWO;
    mg.type = typeGate; mu.type = typeUp; md.type = typeDown;
    auto *own = &c.uploads;
    if ((rc = device_weights(st, wQ, matrix_bytes(typeQ, n0, wO_N), typeQ, &mq.w, own)) ||
        (rc = device_weights(st, wK, matrix_bytes(typeK, n1, wO_N), typeK, &mk.w, own)) ||
        (rc = device_weights(st, wV, matrix_bytes(typeV, n2, wO_N), typeV, &mv.w, own)) ||
        (rc = device_weights(st, wO, matrix_bytes(typeWO, wO_N, wO_K), typeWO, &mo.w, own)) ||
        (rc = device_weights(st, gate, matrix_bytes(typeGate, ffnDim, wO_N), typeGate, &mg.w, own)) ||
        (rc = device_weights(st, up, matrix_bytes(typeUp, ffnDim, wO_N), typeUp, &mu.w, own)) ||
        (rc = device_weights(st, down, matrix_bytes(typeDown, wO_N, ffnDim), typeDown, &md.w, own))) {
        drop_uploads(st, c.uploads);
        return rc;
    }
    c.set = true;
    c.kv_layer = kvLayerIndex;
    c.q = mq; c.k = mk; c.v = mv; c.o = mo; c.gate = mg; c.up = mu; c.down = md;
    c.n0 = n0; c.n1 = wK ? n1 : nKVH * headDim; c.n2 = wV || wK ? (wV ? n2 : c.n1) : nKVH * headDim;
    c.wo_k = wO_K; c.wo_n = wO_N; c.ffn = ffnDim;
    c.nh = nH; c.nkv = nKVH; c.hd = headDim; c.stride = stride;
    c.freq_base = freqBase; c.is_swa = isSwa; c.out_scale = outScale; c.attn_scale = attnScale;
    c.post_attn = hasPostAttnNorm; c.post_ffn = hasPostFfnNorm; c.q_norm = hasQNorm; c.k_norm = hasKNorm;
    c.unit_v = hasUnitVNorm;
    if (layer >= st.num_layers) st.num_layers = layer + 1;
    st.geometry_ready = false;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_register_output(const float *outputNormW, const void *outputW, int typeOutputW, int outputK,
                                int outputN, float cap) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    ALJ_REQUIRE(outputK > 0 && outputN > 0, "register_output: outputK and outputN must be positive");
    int rc = check_mat(outputW, typeOutputW, outputN, outputK, "output");
    if (rc) return rc;
    Mat w;
    w.type = typeOutputW;
    st.out_w = Mat();
    drop_uploads(st, st.out_uploads);
    if ((rc = device_weights(st, outputW, matrix_bytes(typeOutputW, outputN, outputK), typeOutputW, &w.w,
                             &st.out_uploads)))
        return rc;
    if (outputNormW && is_device_ptr(outputNormW)) {
        st.out_norm_owned.release();
        st.out_norm = outputNormW;
    } else if (outputNormW) {
        if (!st.out_norm_owned.ensure(static_cast<size_t>(outputK) * 4))
            return fail(ALJABR_ROCM_ERR_BUFFER, "register_output: cannot allocate");
        if (hipMemcpy(st.out_norm_owned.p, outputNormW, static_cast<size_t>(outputK) * 4, hipMemcpyHostToDevice) !=
            hipSuccess)
            return fail(ALJABR_ROCM_ERR_DEVICE, "register_output: upload failed");
        st.out_norm = st.out_norm_owned.f();
    } else {
        st.out_norm = nullptr;
    }
    st.out_w = w;
    st.out_k = outputK;
    st.out_n = outputN;
    st.cap = cap;
    if (!st.logits.ensure(static_cast<size_t>(outputN) * 4))
        return fail(ALJABR_ROCM_ERR_BUFFER, "register_output: cannot allocate logits");
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_register_token_embd(const void *embdW, int typeEmbdW, int dim, float scale) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    ALJ_REQUIRE(embdW && dim > 0 && std::isfinite(scale) && st.out_n > 0,
                "register_token_embd: weights, dim > 0, a finite scale and a registered output (its vocab)");
    int rc = check_mat(embdW, typeEmbdW, st.out_n, dim, "token_embd");
    if (rc) return rc;
    Mat w;
    w.type = typeEmbdW;
    st.embd = Mat();
    drop_uploads(st, st.embd_uploads);
    if ((rc = device_weights(st, embdW, matrix_bytes(typeEmbdW, st.out_n, dim), typeEmbdW, &w.w, &st.embd_uploads)))
        return rc;
    st.embd = w;
    st.embd_dim = dim;
    st.embd_vocab = st.out_n;
    st.embd_scale = scale;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_decode_step(int pos, int slidingWindow, float eps, const float *x_in, float *logits_out) {
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained(decode_step_locked(st, pos, slidingWindow, eps, x_in, -1, logits_out));
}

int aljabr_rocm_decode_step_token(int pos, int slidingWindow, float eps, int tokenId, float *logits_out) {
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    if (tokenId < 0 || tokenId >= st.embd_vocab || !st.embd.w)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "decode_step_token: token %d outside the registered embedding (%d)",
                    tokenId, st.embd_vocab);
    return drained(decode_step_locked(st, pos, slidingWindow, eps, nullptr, tokenId, logits_out));
}

int aljabr_rocm_set_decode_activation(int activationKind) {
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    ALJ_REQUIRE(activationKind == 1 || activationKind == 2, "set_decode_activation: 1 (SiLU) or 2 (GELU)");
    st.activation = activationKind;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_reset_decode_state(void) {
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    if (aljabr_rocm_is_initialized()) (void)hipDeviceSynchronize();
    st.release_all();
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_wo_ffn_next_qkv_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K,
                                      int wO_N, const float *postAttnW, int hasPostAttnNorm, const float *ffnNormW,
                                      const float *postFfnW, int hasPostFfnNorm, float eps, float outScale,
                                      const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                                      int typeDown, int ffnDim, int activationKind, int hasNext,
                                      const float *nextAttnNormW, float *nextQ, float *nextK, float *nextV,
                                      const void *nextWQ, const void *nextWK, const void *nextWV, int nextTypeQ,
                                      int nextTypeK, int nextTypeV, int nextN0, int nextN1, int nextN2) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        const bool next = hasNext && nextWQ;
        if (next) {
            ALJ_REQUIRE(nextAttnNormW && nextQ && nextN0 > 0 && (!nextWK || (nextK && nextN1 > 0)) &&
                            (!nextWV || (nextV && nextN2 > 0)),
                        "wo_ffn_next_qkv_fused: the next layer's norm, outputs and sizes are required");
        }
        const int qn = next ? std::max(nextN0, std::max(nextWK ? nextN1 : 0, nextWV ? nextN2 : 0)) : 0;
        int rc = adhoc_prepare(st, std::max(wO_N, 1), std::max(wO_K, 1), std::max(ffnDim, 1), qn, 0);
        if (rc) return rc;
        hipStream_t s = current_stream();
        size_t used = 0;
        const AdHoc a{x, attn_full, wO, typeWO, wO_K, wO_N, postAttnW, hasPostAttnNorm, ffnNormW, postFfnW, hasPostFfnNorm,
                      eps, outScale, gateW, upW, downW, typeGate, typeUp, typeDown, ffnDim, activationKind};
        if ((rc = adhoc_layer(st, a, s, used))) return rc;
        if (next) {
            const void *ws[3] = {nextWQ, nextWK, nextWV};
            const int ts[3] = {nextTypeQ, nextTypeK, nextTypeV}, ns[3] = {nextN0, nextN1, nextN2};
            float *outs[3] = {st.q.f(), st.k.f(), st.v.f()};
            float *dst[3] = {nextQ, nextK, nextV};
            float *ys[3];
            const uint8_t *dw[3];
            int yn[3], yt[3], n = 0, idx[3];
            for (int i = 0; i < 3; ++i) {
                if (!ws[i]) continue;
                if ((rc = check_mat(ws[i], ts[i], ns[i], wO_N, "next Q/K/V"))) return rc;
                Mat m;
                if ((rc = device_weights(st, ws[i], matrix_bytes(ts[i], ns[i], wO_N), ts[i], &m.w))) return rc;
                ys[n] = outs[i]; dw[n] = m.w; yn[n] = ns[i]; yt[n] = ts[i]; idx[n++] = i;
            }
            rc = ALJABR_ROCM_OK;
            const float *nw = view_in(st, nextAttnNormW, static_cast<size_t>(wO_N) * 4, used, s, rc);
            if (rc) return rc;
            if ((rc = enqueue_rmsnorm(st.xb.f(), st.x.f(), nw, 1, wO_N, eps))) return rc;
            if ((rc = enqueue_matmul_multi(ys, st.xb.f(), dw, wO_N, yn, yt, n, 1))) return rc;
            for (int j = 0; j < n; ++j)
                if ((rc = copy_out(dst[idx[j]], ys[j], static_cast<size_t>(yn[j]) * 4, s))) return rc;
        }
        if ((rc = copy_out(x, st.x.p, static_cast<size_t>(wO_N) * 4, s))) return rc;
        if ((rc = launch_ok("wo_ffn_fused"))) return rc;
        return sync(s, "wo_ffn_fused");
    }());
}

int aljabr_rocm_wo_ffn_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K, int wO_N,
                             const float *postAttnW, int hasPostAttnNorm, int addOnePostAttn, const float *ffnNormW,
                             int addOneFfnNorm, const float *postFfnW, int hasPostFfnNorm, int addOnePostFfn, float eps,
                             const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                             int typeDown, int ffnDim, int activationKind) {
    (void)addOnePostAttn;
    (void)addOneFfnNorm;
    (void)addOnePostFfn;
    return aljabr_rocm_wo_ffn_next_qkv_fused(x, attn_full, wO, typeWO, wO_K, wO_N, postAttnW, hasPostAttnNorm,
                                             ffnNormW, postFfnW, hasPostFfnNorm, eps, 1.0f, gateW, upW, downW,
                                             typeGate, typeUp, typeDown, ffnDim, activationKind, 0, nullptr, nullptr,
                                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 0);
}

int aljabr_rocm_wo_ffn_logits_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K, int wO_N,
                                    const float *postAttnW, int hasPostAttnNorm, const float *ffnNormW,
                                    const float *postFfnW, int hasPostFfnNorm, float eps, float outScale,
                                    const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                                    int typeDown, int ffnDim, int activationKind, const float *outputNormW,
                                    const void *outputW, int typeOutputW, int outputK, int outputN, float *logits,
                                    float cap) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        ALJ_REQUIRE(outputK > 0 && outputN > 0 && outputK == wO_N && outputNormW && outputW && logits,
                    "wo_ffn_logits_fused: outputK == wO_N, the output norm, weights and logits are required");
        int rc = check_mat(outputW, typeOutputW, outputN, outputK, "output");
        if (rc) return rc;
        if ((rc = adhoc_prepare(st, std::max(wO_N, 1), std::max(wO_K, 1), std::max(ffnDim, 1), 0, outputN))) return rc;
        hipStream_t s = current_stream();
        size_t used = 0;
        const AdHoc a{x, attn_full, wO, typeWO, wO_K, wO_N, postAttnW, hasPostAttnNorm, ffnNormW, postFfnW, hasPostFfnNorm,
                      eps, outScale, gateW, upW, downW, typeGate, typeUp, typeDown, ffnDim, activationKind};
        if ((rc = adhoc_layer(st, a, s, used))) return rc;
        Mat w;
        w.type = typeOutputW;
        if ((rc = device_weights(st, outputW, matrix_bytes(typeOutputW, outputN, outputK), typeOutputW, &w.w)))
            return rc;
        rc = ALJABR_ROCM_OK;
        const float *nw = view_in(st, outputNormW, static_cast<size_t>(outputK) * 4, used, s, rc);
        if (rc) return rc;
        if ((rc = logits_step(st, w, nw, outputK, outputN, cap, eps))) return rc;
        if ((rc = copy_out(logits, st.logits.p, static_cast<size_t>(outputN) * 4, s))) return rc;
        if (x && (rc = copy_out(x, st.x.p, static_cast<size_t>(wO_N) * 4, s))) return rc;
        if ((rc = launch_ok("wo_ffn_logits_fused"))) return rc;
        return sync(s, "wo_ffn_logits_fused");
    }());
}

void aljabr_rocm_wo_ffn_reset_x(void) {}

int aljabr_rocm_wo_ffn_fused_layer_batch(float *x, const float *attn_full, int layer, int batchSize, float eps,
                                         int activationKind) {
    ALJ_CHECK_READY();
    State &st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    return drained([&]() -> int {
        ALJ_REQUIRE(layer >= 0 && layer < st.num_layers && st.layer[layer].set && batchSize > 0 && x && attn_full,
                    "wo_ffn_fused_layer_batch: a registered layer, batchSize > 0, x and attn_full");
        const Layer &c = st.layer[layer];
        if (!st.norm[1].p) return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "wo_ffn_fused_layer_batch: the FFN norm (slot 1) is required");
        int rc = prepare(st, batchSize);
        if (rc) return rc;
        // The activation buffers hold rows of the model width (layer 0's).
        ALJ_REQUIRE(c.wo_n == st.dim, "wo_ffn_fused_layer_batch: layer %d's width %d is not the model width %d", layer,
                    c.wo_n, st.dim);
        const int dim = c.wo_n;
        const float *ffn_norm, *post_attn, *post_ffn;
        if ((rc = slot_row(st, 1, layer, dim, &ffn_norm)) || (rc = slot_row(st, 0, layer, dim, &post_attn)) ||
            (rc = slot_row(st, 2, layer, dim, &post_ffn)))
            return rc;
        if (!c.post_attn) post_attn = nullptr;
        if (!c.post_ffn) post_ffn = nullptr;
        hipStream_t s = current_stream();
        const size_t xb = static_cast<size_t>(batchSize) * dim * 4;
        if ((rc = copy_in(st.x.p, x, xb, s)) ||
            (rc = copy_in(st.att.p, attn_full, static_cast<size_t>(batchSize) * c.wo_k * 4, s)))
            return rc;
        FfnLayer f{c.o, c.gate, c.up, c.down, c.wo_k, dim, c.ffn, post_attn, ffn_norm, post_ffn, c.out_scale};
        if ((rc = wo_ffn(st, f, batchSize, eps, activationKind))) return rc;
        if ((rc = copy_out(x, st.x.p, xb, s))) return rc;
        if ((rc = launch_ok("wo_ffn_fused_layer_batch"))) return rc;
        return sync(s, "wo_ffn_fused_layer_batch");
    }());
}

}  // extern "C"
