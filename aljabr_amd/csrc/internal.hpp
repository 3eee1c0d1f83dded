// internal.hpp - host-side plumbing shared by the C-ABI entry points.
//
// Status codes, the thread-local error message, the calling thread's stream and
// the per-stream scratch arena. Kernels live in the *.hip files that include
// this header; no entry point allocates torch memory or calls back into Python.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/aljabr_rocm.h"

namespace aljabr {

// Records `msg` as this thread's last error and returns `status`.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// ALJABR_ROCM_OK when the library is initialised and the calling thread is
// bound to the library device; otherwise the failing status (message set).
int ensure_ready();

// The calling thread's stream (set_stream override or library-owned stream).
hipStream_t current_stream();

// After enqueuing work: checks the launch, and in synchronous mode waits for
// the stream and reports asynchronous device errors.
int finish_launch(const char *what);

// Device scratch owned by the library for the calling thread's stream; grows
// monotonically. Stream order makes reuse by later calls on the same stream
// safe. Returns nullptr (and records an error) on allocation failure, and
// while the stream is being captured (a graph would keep an address a later
// growth frees). Slots
// are separate buffers: kScratchPartials holds the matrix-core GEMMs' K-slice
// partials, so a caller that keeps its own data in slot 0 across a GEMM call
// is not overwritten.
constexpr int kScratchSlots = 2;
constexpr int kScratchPartials = 1;
void *stream_scratch(size_t bytes, int slot = 0);
// Bytes of stream scratch held for the calling thread's stream (all slots).
size_t stream_scratch_held();

// Number of compute units of the initialised device (for grid sizing).
int device_cu_count();

// Frees the registered whole-step decode model (KV caches, uploads,
// activations); called by aljabr_rocm_shutdown.
void step_state_release();

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// log2 of a power of two, -1 for anything else.
inline int log2_exact(int v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

}  // namespace aljabr

#define ALJ_CHECK_READY()                          \
    do {                                           \
        int _rc = ::aljabr::ensure_ready();        \
        if (_rc != ALJABR_ROCM_OK) return _rc;     \
    } while (0)

#define ALJ_REQUIRE(cond, ...)                                              \
    do {                                                                    \
        if (!(cond)) return ::aljabr::fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, __VA_ARGS__); \
    } while (0)
