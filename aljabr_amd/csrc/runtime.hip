// runtime.hip - lifecycle, device query, streams, memory and errors of the C ABI.
//
// Plays the role of the Metal runtime/buffer layer
// (backend/metal/aljabr-backend-metal/src/main/cpp/metal/aljabr_metal_runtime.m,
// aljabr_metal_buffers.m) for HIP: one context per process bound to one device,
// one non-blocking stream per calling thread, explicit device buffers.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

namespace aljabr {
namespace {

struct Scratch {
    void *ptr = nullptr;
    size_t bytes = 0;
};

struct Context {
    std::mutex mu;
    std::atomic<bool> initialized{false};
    int device = -1;
    int cu_count = 0;
    std::atomic<uint64_t> generation{0};   // bumps on every (re)init so stale thread state is dropped
    std::vector<hipStream_t> owned_streams;                  // one per thread, created lazily
    std::unordered_map<hipStream_t, Scratch[kScratchSlots]> scratch;   // per stream and slot
};

Context &ctx() {
    static Context *c = new Context();   // never destroyed: safe at process exit
    return *c;
}

struct ThreadState {
    uint64_t generation = 0;
    hipStream_t own = nullptr;
    hipStream_t override_stream = nullptr;
    bool has_override = false;
    bool synchronous = true;
    std::string error;
};

ThreadState &tls() {
    thread_local ThreadState t;
    return t;
}

}  // namespace

int fail(int status, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    tls().error = buf;
    return status;
}

static int hip_fail(hipError_t e, int status, const char *what) {
    return fail(status, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

int ensure_ready() {
    Context &c = ctx();
    if (!c.initialized.load(std::memory_order_acquire))
        return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "aljabr_rocm_init has not been called");
    ThreadState &t = tls();
    uint64_t gen = c.generation.load(std::memory_order_acquire);
    if (t.generation != gen) {
        hipError_t e = hipSetDevice(c.device);
        if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipSetDevice");
        t.own = nullptr;
        t.generation = gen;
    }
    if (!t.has_override && t.own == nullptr) {
        hipStream_t s = nullptr;
        hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipStreamCreateWithFlags");
        std::lock_guard<std::mutex> lock(c.mu);
        c.owned_streams.push_back(s);
        t.own = s;
    }
    return ALJABR_ROCM_OK;
}

hipStream_t current_stream() {
    ThreadState &t = tls();
    return t.has_override ? t.override_stream : t.own;
}

int finish_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, what);
    if (tls().synchronous) {
        e = hipStreamSynchronize(current_stream());
        if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, what);
    }
    return ALJABR_ROCM_OK;
}

void *stream_scratch(size_t bytes, int slot) {
    Context &c = ctx();
    hipStream_t s = current_stream();
    // A captured graph would keep this buffer's address while a later,
    // larger request on the stream frees it: work under capture brings its
    // own buffers.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(s, &cs);
    if (ce != hipSuccess || cs != hipStreamCaptureStatusNone) {
        fail(ALJABR_ROCM_ERR_BUFFER, "stream scratch requested while the stream is being captured");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(c.mu);
    Scratch &sc = c.scratch[s][slot];
    if (sc.bytes >= bytes) return sc.ptr;
    // Growing: the old buffer may still be read by queued work on this stream.
    if (sc.ptr) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(sc.ptr);
        sc.ptr = nullptr;
        sc.bytes = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        hip_fail(e, ALJABR_ROCM_ERR_BUFFER, "scratch hipMalloc");
        return nullptr;
    }
    sc.ptr = p;
    sc.bytes = want;
    return p;
}

size_t stream_scratch_held() {
    Context &c = ctx();
    const hipStream_t s = current_stream();
    std::lock_guard<std::mutex> lock(c.mu);
    const auto it = c.scratch.find(s);
    if (it == c.scratch.end()) return 0;
    size_t total = 0;
    for (const Scratch &sc : it->second) total += sc.bytes;
    return total;
}

int device_cu_count() { return ctx().cu_count; }

}  // namespace aljabr

using namespace aljabr;

extern "C" {

int aljabr_rocm_version(void) { return 100; /* 0.1.0 */ }

const char *aljabr_rocm_last_error(void) { return tls().error.c_str(); }

int aljabr_rocm_device_count(int *count) {
    if (!count) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;   // no driver / no GPU: zero devices, not an error
    *count = n;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_device_info_get(int ordinal, aljabr_rocm_device_info *info) {
    if (!info) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "info is null");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || ordinal < 0 || ordinal >= n)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "device ordinal %d out of range (%d devices)", ordinal, n);
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, ordinal);
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipGetDeviceProperties");
    std::memset(info, 0, sizeof(*info));
    std::snprintf(info->name, sizeof(info->name), "%s", p.name);
    std::snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
    info->total_bytes = p.totalGlobalMem;
    info->compute_units = p.multiProcessorCount;
    info->wavefront_size = p.warpSize;
    info->clock_khz = p.clockRate;
    info->memory_clock_khz = p.memoryClockRate;
    info->memory_bus_width = p.memoryBusWidth;
    info->l2_bytes = p.l2CacheSize;
    int rv = 0, dv = 0;
    (void)hipRuntimeGetVersion(&rv);
    (void)hipDriverGetVersion(&dv);
    info->runtime_version = rv;
    info->driver_version = dv;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (hipSetDevice(ordinal) == hipSuccess) {
        size_t fr = 0, tot = 0;
        if (hipMemGetInfo(&fr, &tot) == hipSuccess) info->free_bytes = fr;
        if (cur >= 0) (void)hipSetDevice(cur);
    }
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_init(int ordinal) {
    Context &c = ctx();
    std::lock_guard<std::mutex> lock(c.mu);
    if (c.initialized.load()) {
        if (c.device == ordinal) return ALJABR_ROCM_OK;
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "already initialised on device %d", c.device);
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "no HIP device is visible");
    if (ordinal < 0 || ordinal >= n)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "device ordinal %d out of range (%d devices)", ordinal, n);
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, ordinal);
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipGetDeviceProperties");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "device %d is %s; this library holds gfx950 code only",
                    ordinal, p.gcnArchName);
    e = hipSetDevice(ordinal);
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipSetDevice");
    c.device = ordinal;
    c.cu_count = p.multiProcessorCount;
    c.generation.fetch_add(1);
    c.initialized.store(true, std::memory_order_release);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_is_initialized(void) { return ctx().initialized.load() ? 1 : 0; }

int aljabr_rocm_shutdown(void) {
    Context &c = ctx();
    // The registered decode model's buffers first (its lock is taken before
    // this context's by every path).
    if (c.initialized.load()) step_state_release();
    std::lock_guard<std::mutex> lock(c.mu);
    if (!c.initialized.load()) return ALJABR_ROCM_OK;
    (void)hipSetDevice(c.device);
    (void)hipDeviceSynchronize();
    for (auto &kv : c.scratch)
        for (Scratch &sc : kv.second)
            if (sc.ptr) (void)hipFree(sc.ptr);
    c.scratch.clear();
    for (hipStream_t s : c.owned_streams) (void)hipStreamDestroy(s);
    c.owned_streams.clear();
    c.initialized.store(false);
    c.generation.fetch_add(1);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_set_stream(void *hip_stream) {
    ThreadState &t = tls();
    t.has_override = hip_stream != nullptr;
    t.override_stream = static_cast<hipStream_t>(hip_stream);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_stream_scratch_bytes(size_t *bytes) {
    if (!bytes) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "bytes is null");
    ALJ_CHECK_READY();
    *bytes = stream_scratch_held();
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_get_stream(void **hip_stream) {
    if (!hip_stream) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "hip_stream is null");
    ALJ_CHECK_READY();
    *hip_stream = current_stream();
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_set_sync_mode(int synchronous) {
    tls().synchronous = synchronous != 0;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_synchronize(void) {
    ALJ_CHECK_READY();
    hipError_t e = hipStreamSynchronize(current_stream());
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_DEVICE, "hipStreamSynchronize");
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_alloc(size_t bytes, void **device_ptr) {
    if (!device_ptr) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "device_ptr is null");
    *device_ptr = nullptr;
    ALJ_CHECK_READY();
    if (bytes == 0) return ALJABR_ROCM_OK;
    hipError_t e = hipMalloc(device_ptr, bytes);
    if (e != hipSuccess) {
        *device_ptr = nullptr;
        return hip_fail(e, ALJABR_ROCM_ERR_BUFFER, "hipMalloc");
    }
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_free(void *device_ptr) {
    ALJ_CHECK_READY();
    if (!device_ptr) return ALJABR_ROCM_OK;
    hipError_t e = hipFree(device_ptr);
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_BUFFER, "hipFree");
    return ALJABR_ROCM_OK;
}

static int copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, const char *what) {
    ALJ_CHECK_READY();
    if (bytes == 0) return ALJABR_ROCM_OK;
    if (!dst || !src) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "%s: null pointer", what);
    hipStream_t s = current_stream();
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, s);
    if (e == hipSuccess && kind != hipMemcpyDeviceToDevice) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, ALJABR_ROCM_ERR_BUFFER, what);
    if (kind == hipMemcpyDeviceToDevice) return finish_launch(what);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    return copy(dst, src, bytes, hipMemcpyHostToDevice, "memcpy_h2d");
}

int aljabr_rocm_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, "memcpy_d2h");
}

int aljabr_rocm_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, "memcpy_d2d");
}

}  // extern "C"
