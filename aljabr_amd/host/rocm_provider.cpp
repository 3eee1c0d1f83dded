// rocm_provider.cpp - the ROCm compute provider over the C ABI of
// libaljabr_rocm.so, following the Metal provider's shape:
//   * the library is bound with dlopen/dlsym when a session opens, never at
//     discovery (MTLJ/MetalComputeProvider.java:73-74,101-108;
//     spi/aljabr-spi-core/.../ProviderDiscovery.java:19-25); its path comes
//     from the context key "aljabr.rocm.library", the ALJABR_ROCM_LIBRARY
//     environment variable, or sits next to this library
//     (MTLJ/binding/MetalLibraryDiscovery.java:28);
//   * a non-zero status becomes the exception the Java binding would throw
//     (MTLJ/binding/MetalBinding.java:2135-2144): -2 IllegalArgumentException,
//     -3 UnsupportedOperationException, anything else IllegalStateException;
//   * an op's output storage is allocated first and released again if the
//     op fails (MTLJ/MetalComputeBackend.java:199-237).
// MTLJ = backend/metal/aljabr-backend-metal/src/main/java/tech/kayys/aljabr/backend/metal.
#include "spi.hpp"

#include <dlfcn.h>

#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <regex>
#include <set>

#include "aljabr_rocm.h"

namespace aljabr::spi {

// ---- value types -------------------------------------------------------------
namespace {
std::string require_text(const std::string &v, const char *field) {
    const auto b = v.find_first_not_of(" \t\n\r");
    if (b == std::string::npos) throw IllegalArgumentException(std::string(field) + " must not be blank");
    const auto e = v.find_last_not_of(" \t\n\r");
    return v.substr(b, e - b + 1);
}
std::optional<std::string> normalize(const std::optional<std::string> &v) {
    if (!v) return std::nullopt;
    const auto b = v->find_first_not_of(" \t\n\r");
    if (b == std::string::npos) return std::nullopt;
    const auto e = v->find_last_not_of(" \t\n\r");
    return v->substr(b, e - b + 1);
}
}  // namespace

ProviderContext::ProviderContext(std::string version, std::map<std::string, std::string> config)
    : aljabrVersion(require_text(version, "aljabrVersion")), configuration(std::move(config)) {}

std::optional<std::string> ProviderContext::config(const std::string &key) const {
    auto it = configuration.find(key);
    if (it == configuration.end()) return std::nullopt;
    return it->second;
}

ProviderDescriptor::ProviderDescriptor(std::string id_, std::string version_, std::string api_)
    : id(require_text(id_, "id")), version(require_text(version_, "version")),
      apiCompatibility(require_text(api_, "apiCompatibility")) {
    static const std::regex kId("[a-z0-9][a-z0-9._-]*/[a-z0-9][a-z0-9._-]*");
    if (!std::regex_match(id, kId))
        throw IllegalArgumentException("id must use lowercase namespace/name form: " + id);
}

DeviceDescriptor::DeviceDescriptor(std::string providerId_, std::string deviceId_, std::string name_,
                                   DeviceKind kind_, std::optional<long long> total,
                                   std::optional<long long> free_, std::optional<std::string> vendor_,
                                   std::optional<std::string> arch, std::optional<std::string> driver,
                                   std::optional<std::string> runtime)
    : providerId(require_text(providerId_, "providerId")), deviceId(require_text(deviceId_, "deviceId")),
      name(require_text(name_, "name")), kind(kind_), totalMemoryBytes(total), freeMemoryBytes(free_),
      vendor(normalize(vendor_)), architecture(normalize(arch)), driverVersion(normalize(driver)),
      runtimeVersion(normalize(runtime)) {
    if (total && *total < 0) throw IllegalArgumentException("totalMemoryBytes must be non-negative");
    if (free_ && *free_ < 0) throw IllegalArgumentException("freeMemoryBytes must be non-negative");
    if (total && free_ && *free_ > *total)
        throw IllegalArgumentException("freeMemoryBytes must not exceed totalMemoryBytes");
}

OperationSupportDescriptor::OperationSupportDescriptor(std::string op, OperationSupport s,
                                                       std::optional<std::string> backend)
    : operationId(require_text(op, "operationId")), support(s), effectiveBackendId(normalize(backend)) {
    if (support == OperationSupport::DELEGATED && !effectiveBackendId)
        throw IllegalArgumentException("DELEGATED support requires effectiveBackendId");
}

OperationSupportDescriptor ProviderSession::operationSupport(const std::string &operationId,
                                                             const std::map<std::string, std::string> &) {
    return OperationSupportDescriptor(operationId, OperationSupport::UNKNOWN, std::nullopt);
}

const char *dtype_name(DType t) {
    switch (t) {
    case DType::F32: return "F32";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::I32: return "I32";
    case DType::I8: return "I8";
    case DType::INT8: return "INT8";
    case DType::Q8_0: return "Q8_0";
    case DType::Q4_K: return "Q4_K";
    case DType::Q4_0: return "Q4_0";
    case DType::NF4: return "NF4";
    }
    return "?";
}

long long memory_footprint_bytes(DType t, long long n) {
    switch (t) {
    case DType::F32:
    case DType::I32: return 4 * n;
    case DType::F16:
    case DType::BF16: return 2 * n;
    case DType::I8:
    case DType::INT8: return n;
    case DType::Q8_0: return (n + 31) / 32 * 34;
    case DType::Q4_0: return (n + 31) / 32 * 18;
    case DType::Q4_K: return (n + 255) / 256 * 144;
    case DType::NF4: return (n + 1) / 2;
    }
    return 0;
}

// ---- Tensor -----------------------------------------------------------------
Tensor::Tensor(std::vector<long long> shape, DType dtype, TensorStorage *storage, TensorStorage *scales,
               int blockSize)
    : shape_(std::move(shape)), dtype_(dtype), storage_(storage), scales_(scales), block_size_(blockSize) {}

Tensor::Tensor(Tensor &&o) noexcept { *this = std::move(o); }

Tensor &Tensor::operator=(Tensor &&o) noexcept {
    if (this != &o) {
        close();
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        storage_ = o.storage_;
        scales_ = o.scales_;
        block_size_ = o.block_size_;
        o.storage_ = o.scales_ = nullptr;
    }
    return *this;
}

Tensor::~Tensor() {
    try {
        close();
    } catch (...) {
    }
}

long long Tensor::numel() const {
    long long n = 1;
    for (long long d : shape_) n *= d;
    return n;
}

void Tensor::close() {
    if (storage_) storage_->release();
    if (scales_) scales_->release();
    storage_ = scales_ = nullptr;
}

namespace {

// ---- the C ABI, bound at session open --------------------------------------
struct Binding {
    void *handle = nullptr;
    decltype(&aljabr_rocm_init) init = nullptr;
    decltype(&aljabr_rocm_shutdown) shutdown = nullptr;
    decltype(&aljabr_rocm_device_count) device_count = nullptr;
    decltype(&aljabr_rocm_device_info_get) device_info_get = nullptr;
    decltype(&aljabr_rocm_last_error) last_error = nullptr;
    decltype(&aljabr_rocm_alloc) alloc = nullptr;
    decltype(&aljabr_rocm_free) free = nullptr;
    decltype(&aljabr_rocm_memcpy_h2d) h2d = nullptr;
    decltype(&aljabr_rocm_memcpy_d2h) d2h = nullptr;
    decltype(&aljabr_rocm_memcpy_d2d) d2d = nullptr;
    decltype(&aljabr_rocm_matvec_tb_batch_nf4) matvec_nf4 = nullptr;
    decltype(&aljabr_rocm_matvec_tb_batch) matvec_batch = nullptr;
    decltype(&aljabr_rocm_attention_gqa) attention_gqa = nullptr;
    decltype(&aljabr_rocm_rmsnorm) rmsnorm = nullptr;
    decltype(&aljabr_rocm_rope) rope = nullptr;
    decltype(&aljabr_rocm_swiglu) swiglu = nullptr;
    decltype(&aljabr_rocm_add_inplace) add_inplace = nullptr;
};

std::mutex g_binding_mutex;
Binding *g_binding = nullptr;                  // process-wide, as MetalBinding:49-51

template <typename F>
void bind_symbol(void *h, const char *name, F &slot) {
    void *p = dlsym(h, name);
    if (!p) throw ProviderException(std::string("ROCm library lacks symbol ") + name);
    slot = reinterpret_cast<F>(p);
}

std::string default_library_path() {
    Dl_info info{};
    if (dladdr(reinterpret_cast<void *>(&default_library_path), &info) && info.dli_fname) {
        std::string self(info.dli_fname);
        auto slash = self.rfind('/');
        if (slash != std::string::npos) return self.substr(0, slash + 1) + "libaljabr_rocm.so";
    }
    return "libaljabr_rocm.so";
}

Binding &binding(const std::string &path) {
    std::lock_guard<std::mutex> lock(g_binding_mutex);
    if (g_binding) return *g_binding;
    void *h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) throw ProviderException("cannot load ROCm library " + path + ": " + dlerror());
    auto *b = new Binding();
    b->handle = h;
    bind_symbol(h, "aljabr_rocm_init", b->init);
    bind_symbol(h, "aljabr_rocm_shutdown", b->shutdown);
    bind_symbol(h, "aljabr_rocm_device_count", b->device_count);
    bind_symbol(h, "aljabr_rocm_device_info_get", b->device_info_get);
    bind_symbol(h, "aljabr_rocm_last_error", b->last_error);
    bind_symbol(h, "aljabr_rocm_alloc", b->alloc);
    bind_symbol(h, "aljabr_rocm_free", b->free);
    bind_symbol(h, "aljabr_rocm_memcpy_h2d", b->h2d);
    bind_symbol(h, "aljabr_rocm_memcpy_d2h", b->d2h);
    bind_symbol(h, "aljabr_rocm_memcpy_d2d", b->d2d);
    bind_symbol(h, "aljabr_rocm_matvec_tb_batch_nf4", b->matvec_nf4);
    bind_symbol(h, "aljabr_rocm_matvec_tb_batch", b->matvec_batch);
    bind_symbol(h, "aljabr_rocm_attention_gqa", b->attention_gqa);
    bind_symbol(h, "aljabr_rocm_rmsnorm", b->rmsnorm);
    bind_symbol(h, "aljabr_rocm_rope", b->rope);
    bind_symbol(h, "aljabr_rocm_swiglu", b->swiglu);
    bind_symbol(h, "aljabr_rocm_add_inplace", b->add_inplace);
    g_binding = b;
    return *b;
}

void check(const Binding &b, int rc, const char *op) {
    if (rc == ALJABR_ROCM_OK) return;
    const char *msg = b.last_error ? b.last_error() : nullptr;
    std::string text = std::string(op) + ": " + (msg && *msg ? msg : "status " + std::to_string(rc));
    if (rc == ALJABR_ROCM_ERR_BAD_ARGUMENT) throw IllegalArgumentException(text);
    if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) throw UnsupportedOperationException(text);
    throw IllegalStateException(text + " (status " + std::to_string(rc) + ")");
}

// ---- device storage ------------------------------------------------------------
class DeviceStorage final : public TensorStorage {
public:
    DeviceStorage(const Binding &b, long long bytes) : b_(b), bytes_(bytes) {
        if (bytes < 0) throw IllegalArgumentException("Invalid storage size: " + std::to_string(bytes));
        check(b_, b_.alloc(static_cast<size_t>(bytes > 0 ? bytes : 1), &ptr_), "allocateStorage");
    }
    long long sizeBytes() const override { return bytes_; }
    void retain() override {
        long long r = refs_.load();
        do {
            if (r <= 0) throw IllegalStateException("storage already released");
        } while (!refs_.compare_exchange_weak(r, r + 1));
    }
    void release() override {
        long long r = refs_.load();
        do {
            if (r <= 0) throw IllegalStateException("storage has no live reference");
        } while (!refs_.compare_exchange_weak(r, r - 1));
        if (r == 1) {
            b_.free(ptr_);
            ptr_ = nullptr;
            delete this;
        }
    }
    void *ptr() const { return ptr_; }

private:
    ~DeviceStorage() override = default;
    const Binding &b_;
    long long bytes_;
    void *ptr_ = nullptr;
    std::atomic<long long> refs_{1};
};

DeviceStorage *device_storage(TensorStorage *s, const char *what) {
    auto *d = dynamic_cast<DeviceStorage *>(s);
    if (!d) throw IllegalArgumentException(std::string(what) + " must be storage of this ROCm backend");
    return d;
}

void *dptr(const Tensor &t, const char *what) {
    if (!t.valid()) throw IllegalArgumentException(std::string(what) + " must not be null");
    return device_storage(t.storage(), what)->ptr();
}

// Output storage owned by the result only after the op succeeds.
struct PendingOutput {
    DeviceStorage *s;
    explicit PendingOutput(DeviceStorage *p) : s(p) {}
    ~PendingOutput() {
        if (s) s->release();
    }
    DeviceStorage *take() {
        auto *p = s;
        s = nullptr;
        return p;
    }
};

// ---- backend ---------------------------------------------------------------------
class RocmComputeBackend final : public ComputeBackend {
public:
    explicit RocmComputeBackend(const Binding &b) : b_(b) {}

    void close() override { closed_ = true; }
    DeviceType deviceType() const override { return DeviceType::ROCM; }

    TensorStorage *allocateStorage(long long sizeBytes) override {
        live();
        return new DeviceStorage(b_, sizeBytes);
    }

    void copyFromHost(TensorStorage *destination, const void *source, long long sizeBytes) override {
        live();
        auto *d = device_storage(destination, "destination");
        if (sizeBytes < 0 || sizeBytes > d->sizeBytes())
            throw IllegalArgumentException("Invalid host copy size: " + std::to_string(sizeBytes));
        if (sizeBytes == 0) return;
        if (!source) throw IllegalArgumentException("source must not be null");
        check(b_, b_.h2d(d->ptr(), source, static_cast<size_t>(sizeBytes)), "copyFromHost");
    }

    void copyToHost(void *destination, TensorStorage *source, long long sizeBytes) override {
        live();
        auto *s = device_storage(source, "source");
        if (sizeBytes < 0 || sizeBytes > s->sizeBytes())
            throw IllegalArgumentException("Invalid host copy size: " + std::to_string(sizeBytes));
        if (sizeBytes == 0) return;
        if (!destination) throw IllegalArgumentException("destination must not be null");
        check(b_, b_.d2h(destination, s->ptr(), static_cast<size_t>(sizeBytes)), "copyToHost");
    }

    Tensor matmul(const Tensor &a, const Tensor &b) override {
        live();
        if (!a.valid() || !b.valid()) throw IllegalArgumentException("matmul operands must not be null");
        if (a.dtype() != DType::F32) throw UnsupportedOperationException("ROCm matmul needs F32 activations");
        if (a.rank() < 1 || b.rank() != 2) throw IllegalArgumentException("matmul expects a[..., K] and b[N, K]");
        const long long K = a.dim(a.rank() - 1), N = b.dim(0);
        if (b.dim(1) != K)
            throw IllegalArgumentException("matmul inner dimensions differ: a has K=" + std::to_string(K) +
                                           ", b has " + std::to_string(b.dim(1)));
        const long long M = a.numel() / K;
        if (M <= 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
            throw IllegalArgumentException("matmul dimensions out of range");
        PendingOutput out(new DeviceStorage(b_, M * N * 4));
        const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
        switch (b.dtype()) {
        case DType::NF4: {
            if (!b.scales() || b.blockSize() <= 0)
                throw IllegalArgumentException("NF4 weight needs its absmax scales and block size");
            check(b_, b_.matvec_nf4(out.s->ptr(), dptr(a, "a"), dptr(b, "b"),
                                    device_storage(b.scales(), "scales")->ptr(), k, n, b.blockSize(), m),
                  "matmul");
            break;
        }
        case DType::Q4_0:
        case DType::Q8_0:
        case DType::F16: {
            const int type = b.dtype() == DType::Q4_0 ? ALJABR_ROCM_TYPE_Q4_0
                             : b.dtype() == DType::Q8_0 ? ALJABR_ROCM_TYPE_Q8_0 : ALJABR_ROCM_TYPE_F16;
            check(b_, b_.matvec_batch(out.s->ptr(), dptr(a, "a"), dptr(b, "b"), k, n, type, m), "matmul");
            break;
        }
        default:
            throw UnsupportedOperationException(std::string("ROCm matmul does not support weight dtype ") +
                                                dtype_name(b.dtype()));
        }
        std::vector<long long> shape(a.shape().begin(), a.shape().end() - 1);
        shape.push_back(N);
        return Tensor(shape, DType::F32, out.take());
    }

    // Shape and mask rules of CpuBackend.attentionGqa (CPU/CpuBackend.java:1546-1585).
    Tensor attentionGqa(const Tensor &Q, const Tensor &K, const Tensor &V, const Tensor *mask, bool causal) override {
        live();
        if (!Q.valid() || !K.valid() || !V.valid())
            throw IllegalArgumentException("attention Q, K, and V must not be null");
        if (Q.dtype() != DType::F32 || (K.dtype() != DType::F32 && K.dtype() != DType::F16) ||
            V.dtype() != K.dtype())
            throw UnsupportedOperationException("ROCm attention supports F32 Q with F32 or F16 K/V");
        if (Q.rank() != 4 || K.rank() != 4 || V.rank() != 4)
            throw IllegalArgumentException("GQA expects rank-4 [B,H,S,D] Q/K/V tensors");
        const long long B = Q.dim(0), Hq = Q.dim(1), Sq = Q.dim(2), D = Q.dim(3), Hkv = K.dim(1), Sk = K.dim(2);
        if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || D <= 0 || Hq % Hkv != 0 || K.dim(0) != B ||
            V.dim(0) != B || K.dim(3) != D || V.dim(1) != Hkv || V.dim(2) != Sk || V.dim(3) != D)
            throw IllegalArgumentException("GQA expects Q[B,Hq,Sq,D], K/V[B,Hkv,Sk,D] with Hq divisible by Hkv");
        if (mask && mask->valid() &&
            (mask->dtype() != DType::F32 || mask->rank() != 2 || mask->dim(0) != Sq || mask->dim(1) != Sk))
            throw IllegalArgumentException("GQA additive attention mask must be F32 [queryLength, keyLength] on this backend");
        PendingOutput out(new DeviceStorage(b_, B * Hq * Sq * D * 4));
        const void *mp = mask && mask->valid() ? dptr(*mask, "mask") : nullptr;
        check(b_, b_.attention_gqa(out.s->ptr(), dptr(Q, "Q"), dptr(K, "K"), dptr(V, "V"), mp,
                                   static_cast<int>(B), static_cast<int>(Hq), static_cast<int>(Hkv),
                                   static_cast<int>(Sq), static_cast<int>(Sk), static_cast<int>(D),
                                   K.dtype() == DType::F16 ? ALJABR_ROCM_TYPE_F16 : ALJABR_ROCM_TYPE_F32, 0.0f,
                                   causal ? 1 : 0),
              "attentionGqa");
        return Tensor({B, Hq, Sq, D}, DType::F32, out.take());
    }

    // CpuBackend.rmsNorm rules (CPU/CpuBackend.java:781-800,838-842).
    Tensor rmsNorm(const Tensor &input, const Tensor &weight, float eps) override {
        live();
        if (!input.valid() || !weight.valid()) throw IllegalArgumentException("input and weight must not be null");
        if (input.dtype() != DType::F32 || weight.dtype() != DType::F32)
            throw UnsupportedOperationException("ROCm RMSNorm supports F32 tensors only");
        if (!std::isfinite(eps) || eps < 0.0f)
            throw IllegalArgumentException("Normalization epsilon must be finite and non-negative");
        if (weight.rank() != 1) throw IllegalArgumentException("RMSNorm weight must be a rank-1 vector");
        const long long H = weight.dim(0);
        if (H <= 0 || input.rank() == 0 || input.dim(input.rank() - 1) != H)
            throw IllegalArgumentException("RMSNorm weight length must match the input's final dimension");
        const long long rows = input.numel() / H;
        PendingOutput out(new DeviceStorage(b_, input.numel() * 4));
        if (rows > 0)
            check(b_, b_.rmsnorm(out.s->ptr(), dptr(input, "input"), dptr(weight, "weight"), static_cast<int>(rows),
                                 static_cast<int>(H), eps),
                  "rmsNorm");
        return Tensor(input.shape(), DType::F32, out.take());
    }

    // CpuBackend.applyRoPE(input, posOffset, freqBase, isNeox) rules
    // (CPU/CpuBackend.java:921-979). The kernel rotates pairs (i, i + D/2),
    // the NeoX pairing; the interleaved pairing is not implemented here.
    Tensor applyRoPE(const Tensor &input, int posOffset, float freqBase, bool isNeox) override {
        live();
        if (!input.valid()) throw IllegalArgumentException("input must not be null");
        if (input.dtype() != DType::F32) throw UnsupportedOperationException("ROCm RoPE supports F32 tensors only");
        if (input.rank() != 4) throw IllegalArgumentException("RoPE expects [batch, heads, sequence, headDim]");
        if (posOffset < 0 || !std::isfinite(freqBase) || freqBase <= 1.0f)
            throw IllegalArgumentException("posOffset must be non-negative and freqBase must be finite and > 1");
        const long long B = input.dim(0), H = input.dim(1), S = input.dim(2), D = input.dim(3);
        if (B <= 0 || H <= 0 || S <= 0 || D <= 0 || (D & 1))
            throw IllegalArgumentException("RoPE requires positive dimensions and an even headDim");
        if (!isNeox) throw UnsupportedOperationException("ROCm RoPE implements the NeoX (split-half) pairing only");
        const long long rows = B * H * S;
        PendingOutput out(new DeviceStorage(b_, input.numel() * 4));
        check(b_, b_.d2d(out.s->ptr(), dptr(input, "input"), static_cast<size_t>(input.numel() * 4)), "applyRoPE");
        // One position per (b, h, s) row: posOffset + s.
        std::vector<int32_t> pos(static_cast<size_t>(rows));
        for (long long r = 0; r < rows; ++r) pos[static_cast<size_t>(r)] = static_cast<int32_t>(posOffset + r % S);
        DeviceStorage *ps = new DeviceStorage(b_, rows * 4);
        PendingOutput pos_guard(ps);
        check(b_, b_.h2d(ps->ptr(), pos.data(), pos.size() * 4), "applyRoPE");
        check(b_, b_.rope(out.s->ptr(), ps->ptr(), static_cast<int>(rows), 1, static_cast<int>(D), freqBase),
              "applyRoPE");
        return Tensor(input.shape(), DType::F32, out.take());
    }

    Tensor add(const Tensor &a, const Tensor &b) override {
        live();
        same_f32("add", a, b);
        PendingOutput out(new DeviceStorage(b_, a.numel() * 4));
        check(b_, b_.d2d(out.s->ptr(), dptr(a, "a"), static_cast<size_t>(a.numel() * 4)), "add");
        check(b_, b_.add_inplace(out.s->ptr(), dptr(b, "b"), a.numel()), "add");
        return Tensor(a.shape(), DType::F32, out.take());
    }

    Tensor siluMul(const Tensor &gate, const Tensor &up) override {
        live();
        same_f32("siluMul", gate, up);
        PendingOutput out(new DeviceStorage(b_, gate.numel() * 4));
        check(b_, b_.swiglu(out.s->ptr(), dptr(gate, "gate"), dptr(up, "up"), gate.numel()), "siluMul");
        return Tensor(gate.shape(), DType::F32, out.take());
    }

private:
    void live() const {
        if (closed_) throw IllegalStateException("ROCm compute backend is closed");
    }
    static void same_f32(const char *op, const Tensor &a, const Tensor &b) {
        if (!a.valid() || !b.valid()) throw IllegalArgumentException(std::string(op) + " operands must not be null");
        if (a.dtype() != DType::F32 || b.dtype() != DType::F32)
            throw UnsupportedOperationException(std::string("ROCm ") + op + " supports F32 tensors only");
        if (a.shape() != b.shape()) throw UnsupportedOperationException(std::string("ROCm ") + op + " does not broadcast");
    }

    const Binding &b_;
    std::atomic<bool> closed_{false};
};

// ---- session and provider --------------------------------------------------------
constexpr const char *kProviderId = "andalus/rocm";
constexpr const char *kBackendId = "rocm-default";

class RocmProviderSession final : public ProviderSession {
public:
    RocmProviderSession(DeviceDescriptor device, Binding &b, std::shared_ptr<std::atomic<bool>> provider_open)
        : device_(std::move(device)), b_(b), backend_(std::make_unique<RocmComputeBackend>(b)),
          provider_open_(std::move(provider_open)) {}
    ~RocmProviderSession() override {
        try {
            close();
        } catch (...) {
        }
    }

    const DeviceDescriptor &device() const override { return device_; }

    std::map<std::string, ComputeBackend *> computeBackends() override {
        std::lock_guard<std::mutex> lock(mu_);
        close_if_provider_closed();
        if (closed_) throw IllegalStateException("ROCm provider session is closed");
        return {{kBackendId, backend_.get()}};
    }

    // Conservative, as MetalComputeBackend.operationSupport (MTLJ/MetalComputeBackend.java:306-370):
    // NATIVE only where a kernel exists for the requested dtypes.
    OperationSupportDescriptor operationSupport(const std::string &operationId,
                                                const std::map<std::string, std::string> &c) override {
        std::lock_guard<std::mutex> lock(mu_);
        close_if_provider_closed();
        if (closed_) throw IllegalStateException("ROCm provider session is closed");
        const std::string op = require_text(operationId, "operationId");
        auto get = [&](const char *k, const std::string &d) {
            auto it = c.find(k);
            std::string v = it == c.end() ? d : it->second;
            for (auto &ch : v) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
            return v;
        };
        const std::string dtype = get("dtype", "");
        bool native = false;
        if (op == "tensor.matmul") {
            const std::string in = get("inputDtype", dtype), w = get("weightDtype", dtype);
            native = in == "f32" && (w == "nf4" || w == "q4_0" || w == "q8_0" || w == "f16");
        } else if (op == "tensor.attention") {
            native = dtype == "f32" || dtype == "f16";
        } else if (op == "tensor.rms_norm" || op == "tensor.rope" || op == "tensor.add") {
            native = dtype == "f32";
        }
        if (native) return OperationSupportDescriptor(op, OperationSupport::NATIVE, std::nullopt);
        static const std::set<std::string> known = {
            "tensor.add", "tensor.sub", "tensor.mul", "tensor.div", "tensor.add_scalar", "tensor.matmul",
            "tensor.reshape", "tensor.attention", "tensor.softmax", "tensor.slice", "tensor.split", "tensor.pow",
            "tensor.mean", "tensor.abs", "tensor.cast", "tensor.to", "tensor.zeros_like", "tensor.sqrt",
            "tensor.relu", "tensor.sigmoid", "tensor.tanh", "tensor.log", "tensor.exp", "tensor.silu",
            "tensor.flatten", "tensor.unsqueeze", "tensor.squeeze", "tensor.transpose", "tensor.gelu",
            "tensor.log_softmax", "tensor.sum", "tensor.max", "tensor.layer_norm", "tensor.rms_norm",
            "tensor.embedding", "tensor.rope", "tensor.cat"};
        return OperationSupportDescriptor(op, known.count(op) ? OperationSupport::UNSUPPORTED : OperationSupport::UNKNOWN,
                                          std::nullopt);
    }

    void close() override {
        std::lock_guard<std::mutex> lock(mu_);
        if (closed_) return;
        closed_ = true;
        backend_->close();
    }

private:
    // Provider closure closes the sessions it opened (AljabrProvider.java:18-30).
    void close_if_provider_closed() {
        if (!closed_ && !provider_open_->load()) {
            closed_ = true;
            backend_->close();
        }
    }

    DeviceDescriptor device_;
    Binding &b_;
    std::unique_ptr<RocmComputeBackend> backend_;
    std::shared_ptr<std::atomic<bool>> provider_open_;
    std::mutex mu_;
    bool closed_ = false;
};

class RocmComputeProvider final : public ComputeProvider {
public:
    RocmComputeProvider() : descriptor_(kProviderId, "0.1.0", ">=0.1.0 <1.0.0") {}
    ~RocmComputeProvider() override {
        try {
            close();
        } catch (...) {
        }
    }

    const ProviderDescriptor &descriptor() const override { return descriptor_; }

    void initialize(const ProviderContext &context) override {
        std::lock_guard<std::mutex> lock(mu_);
        if (closed_) throw ProviderException("ROCm provider is closed");
        if (initialized_) throw ProviderException("ROCm provider is already initialized");
        if (auto p = context.config("aljabr.rocm.library")) library_ = *p;
        initialized_ = true;
    }

    std::vector<DeviceDescriptor> devices() override {
        std::lock_guard<std::mutex> lock(mu_);
        if (closed_) throw ProviderException("ROCm provider is closed");
        if (!initialized_) throw ProviderException("ROCm provider has not been initialized");
        Binding &b = binding(library_path());
        int n = 0;
        check(b, b.device_count(&n), "devices");
        std::vector<DeviceDescriptor> out;
        for (int i = 0; i < n; ++i) {
            aljabr_rocm_device_info info{};
            if (b.device_info_get(i, &info) != ALJABR_ROCM_OK) continue;
            std::string arch(info.arch);
            arch = arch.substr(0, arch.find(':'));
            out.emplace_back(kProviderId, "rocm:" + std::to_string(i), info.name[0] ? info.name : "AMD GPU",
                             DeviceKind::GPU, static_cast<long long>(info.total_bytes),
                             static_cast<long long>(info.free_bytes), std::string("AMD"), arch,
                             std::to_string(info.driver_version), std::to_string(info.runtime_version));
        }
        return out;
    }

    std::unique_ptr<ProviderSession> openSession(const DeviceDescriptor &device) override {
        std::lock_guard<std::mutex> lock(mu_);
        if (closed_) throw ProviderException("ROCm provider is closed");
        if (!initialized_) throw ProviderException("ROCm provider has not been initialized");
        if (device.providerId != kProviderId)
            throw ProviderException(std::string("Device does not belong to provider ") + kProviderId + ": " +
                                    device.deviceId);
        const std::string prefix = "rocm:";
        if (device.deviceId.compare(0, prefix.size(), prefix) != 0)
            throw ProviderException("Unknown ROCm device id: " + device.deviceId);
        int ordinal = -1;
        try {
            ordinal = std::stoi(device.deviceId.substr(prefix.size()));
        } catch (...) {
            throw ProviderException("Unknown ROCm device id: " + device.deviceId);
        }
        Binding &b = binding(library_path());
        const int rc = b.init(ordinal);
        if (rc != ALJABR_ROCM_OK)
            throw ProviderException(std::string("cannot open ROCm device ") + device.deviceId + ": " + b.last_error());
        return std::make_unique<RocmProviderSession>(device, b, open_);
    }

    void close() override {
        std::lock_guard<std::mutex> lock(mu_);
        closed_ = true;
        open_->store(false);
    }

private:
    std::string library_path() const {
        if (!library_.empty()) return library_;
        if (const char *e = std::getenv("ALJABR_ROCM_LIBRARY"); e && *e) return e;
        return default_library_path();
    }

    ProviderDescriptor descriptor_;
    std::mutex mu_;
    bool initialized_ = false, closed_ = false;
    std::string library_;
    std::shared_ptr<std::atomic<bool>> open_ = std::make_shared<std::atomic<bool>>(true);
};

}  // namespace

std::unique_ptr<ComputeProvider> make_rocm_provider() { return std::make_unique<RocmComputeProvider>(); }

}  // namespace aljabr::spi
