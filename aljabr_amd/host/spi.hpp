// spi.hpp - C++ mirror of the part of Aljabr's Backend SPI that the ROCm
// provider implements: provider lifecycle (AljabrProvider / ComputeProvider /
// ProviderSession), device and operation-support descriptors, and the
// ComputeBackend operations on the quantized-inference path. Names, argument
// meaning and error behaviour follow the Java interfaces they stand for, so a
// caller (or a test) reads like the reference; Java exceptions map to
// std exceptions of the same name in this namespace.
//
// Reference (relative to the andalus-ai/aljabr tree):
//   spi/aljabr-spi-core/src/main/java/tech/kayys/aljabr/spi/provider/
//     AljabrProvider.java:18-30, DeviceDescriptor.java:10-37, DeviceKind.java,
//     ProviderDescriptor.java, ProviderContext.java, OperationSupport.java,
//     OperationSupportDescriptor.java
//   spi/aljabr-spi-compute/src/main/java/tech/kayys/aljabr/spi/compute/
//     ComputeProvider.java:16-29, ProviderSession.java:15-96
//   plugins/ml/aljabr-tensor/src/main/java/tech/kayys/aljabr/core/
//     backend/ComputeBackend.java:35-426, memory/TensorStorage.java:3-41,
//     tensor/DType.java:13-50
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace aljabr::spi {

// ---- exceptions (Java names) ----------------------------------------------
struct ProviderException : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct IllegalArgumentException : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct IllegalStateException : std::logic_error {
    using std::logic_error::logic_error;
};
struct UnsupportedOperationException : std::logic_error {
    using std::logic_error::logic_error;
};

// ---- descriptors -------------------------------------------------------------
enum class DeviceKind { CPU, GPU, ACCELERATOR, OTHER };
enum class OperationSupport { NATIVE, DELEGATED, EMULATED, UNSUPPORTED, UNKNOWN };

// ProviderContext.java: aljabrVersion must not be blank.
struct ProviderContext {
    std::string aljabrVersion;
    std::map<std::string, std::string> configuration;
    ProviderContext(std::string version, std::map<std::string, std::string> config);
    std::optional<std::string> config(const std::string &key) const;
};

// ProviderDescriptor.java: id is lowercase "namespace/name".
struct ProviderDescriptor {
    std::string id, version, apiCompatibility;
    ProviderDescriptor(std::string id, std::string version, std::string apiCompatibility);
};

// DeviceDescriptor.java:10-37, including its validation rules.
struct DeviceDescriptor {
    std::string providerId, deviceId, name;
    DeviceKind kind;
    std::optional<long long> totalMemoryBytes, freeMemoryBytes;
    std::optional<std::string> vendor, architecture, driverVersion, runtimeVersion;
    DeviceDescriptor(std::string providerId, std::string deviceId, std::string name, DeviceKind kind,
                     std::optional<long long> totalMemoryBytes, std::optional<long long> freeMemoryBytes,
                     std::optional<std::string> vendor, std::optional<std::string> architecture,
                     std::optional<std::string> driverVersion, std::optional<std::string> runtimeVersion);
};

// OperationSupportDescriptor.java: DELEGATED requires effectiveBackendId.
struct OperationSupportDescriptor {
    std::string operationId;
    OperationSupport support;
    std::optional<std::string> effectiveBackendId;
    OperationSupportDescriptor(std::string operationId, OperationSupport support,
                               std::optional<std::string> effectiveBackendId);
};

// ---- tensors -------------------------------------------------------------------
// DType.java:13-50 plus NF4, which the reference does not have: an NF4 tensor
// of logical shape [N, K] carries its codes (N*K/2 bytes, high nibble = even
// element) in storage() and its fp32 absmax array (N*K/blockSize floats) in
// scales().
enum class DType { F32, F16, BF16, I32, I8, INT8, Q8_0, Q4_K, Q4_0, NF4 };
enum class DeviceType { CPU, ROCM };

const char *dtype_name(DType t);
// Bytes of `numel` elements (DType.memoryFootprintBytes); NF4 counts codes only.
long long memory_footprint_bytes(DType t, long long numel);

// TensorStorage.java:3-41: reference-counted storage. retain() adds an owner,
// release() drops one; the final release ends the lifetime. Both throw
// IllegalStateException once the storage is released.
class TensorStorage {
public:
    virtual ~TensorStorage() = default;
    virtual long long sizeBytes() const = 0;
    virtual void retain() = 0;
    virtual void release() = 0;
};

// A tensor owns one reference to its storage (and to its scales, for NF4).
class Tensor {
public:
    Tensor() = default;
    Tensor(std::vector<long long> shape, DType dtype, TensorStorage *storage, TensorStorage *scales = nullptr,
           int blockSize = 0);
    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;
    Tensor(Tensor &&o) noexcept;
    Tensor &operator=(Tensor &&o) noexcept;
    ~Tensor();

    const std::vector<long long> &shape() const { return shape_; }
    long long dim(int i) const { return shape_.at(static_cast<size_t>(i)); }
    int rank() const { return static_cast<int>(shape_.size()); }
    long long numel() const;
    DType dtype() const { return dtype_; }
    TensorStorage *storage() const { return storage_; }   // borrowed
    TensorStorage *scales() const { return scales_; }     // borrowed (NF4)
    int blockSize() const { return block_size_; }
    bool valid() const { return storage_ != nullptr; }
    void close();                                          // releases the owned references

private:
    std::vector<long long> shape_;
    DType dtype_ = DType::F32;
    TensorStorage *storage_ = nullptr;
    TensorStorage *scales_ = nullptr;
    int block_size_ = 0;
};

// ComputeBackend.java: the operations on the quantized-inference path. The
// rest of the interface (conv, pooling, losses, ...) is not implemented here;
// operationSupport() reports it so that the fallback policy can route it.
class ComputeBackend {
public:
    virtual ~ComputeBackend() = default;
    virtual void close() = 0;
    virtual DeviceType deviceType() const = 0;
    // Storage with one reference owned by the caller (TensorAllocator contract).
    virtual TensorStorage *allocateStorage(long long sizeBytes) = 0;
    virtual void copyFromHost(TensorStorage *destination, const void *source, long long sizeBytes) = 0;
    // The reverse direction (Java copies into host-accessible storage with copyInto).
    virtual void copyToHost(void *destination, TensorStorage *source, long long sizeBytes) = 0;
    // a [M, K] F32 times b [N, K] (NF4, Q4_0, Q8_0 or F16, "transposed right")
    // -> [M, N] F32.
    virtual Tensor matmul(const Tensor &a, const Tensor &b) = 0;
    // Q [B, Hq, Sq, D] F32, K/V [B, Hkv, Sk, D] F32 or F16, additive mask
    // [Sq, Sk] F32 or null -> [B, Hq, Sq, D] F32.
    virtual Tensor attentionGqa(const Tensor &Q, const Tensor &K, const Tensor &V, const Tensor *additiveMask,
                                bool causal) = 0;
    virtual Tensor rmsNorm(const Tensor &input, const Tensor &weight, float eps) = 0;
    // input [B, H, S, D] F32, positions posOffset + s.
    virtual Tensor applyRoPE(const Tensor &input, int posOffset, float freqBase, bool isNeox) = 0;
    virtual Tensor add(const Tensor &a, const Tensor &b) = 0;
    // silu(gate) * up, the decode step's fused SwiGLU (silu followed by mul).
    virtual Tensor siluMul(const Tensor &gate, const Tensor &up) = 0;
};

// ProviderSession.java:15-96.
class ProviderSession {
public:
    virtual ~ProviderSession() = default;
    virtual const DeviceDescriptor &device() const = 0;
    // Immutable view; throws IllegalStateException after close().
    virtual std::map<std::string, ComputeBackend *> computeBackends() = 0;
    virtual OperationSupportDescriptor operationSupport(const std::string &operationId,
                                                        const std::map<std::string, std::string> &constraints);
    // Terminal and idempotent.
    virtual void close() = 0;
};

// AljabrProvider.java:18-30.
class AljabrProvider {
public:
    virtual ~AljabrProvider() = default;
    virtual const ProviderDescriptor &descriptor() const = 0;
    virtual void initialize(const ProviderContext &context) = 0;   // at most once
    virtual void close() = 0;                                      // terminal, idempotent
};

// ComputeProvider.java:16-29.
class ComputeProvider : public AljabrProvider {
public:
    virtual std::vector<DeviceDescriptor> devices() = 0;
    // Rejects a descriptor whose providerId is not this provider's.
    virtual std::unique_ptr<ProviderSession> openSession(const DeviceDescriptor &device) = 0;
};

// The ROCm provider ("andalus/rocm"). It loads nothing at construction
// (discovery must not load native code, ProviderDiscovery.java:19-25): the
// device runtime starts in openSession.
std::unique_ptr<ComputeProvider> make_rocm_provider();

}  // namespace aljabr::spi
