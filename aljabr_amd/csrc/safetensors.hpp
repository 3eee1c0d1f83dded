// safetensors.hpp - a safetensors file mapped read-only and parsed: the
// loader behind aljabr_rocm_safetensors_* and aljabr_rocm_llama_create_safetensors.
// Restates the layout the reference's parser reads
// (engine/safetensor/aljabr-safetensor-loader/.../SafetensorHeaderParser.java:
// 13-24,127-160): a little-endian u64 header length N (at most 100 MiB), N
// bytes of UTF-8 JSON mapping each tensor name to {"dtype", "shape",
// "data_offsets": [begin, end]} (offsets relative to the data that follows
// the header) plus an optional "__metadata__" string map. Every tensor's
// range must lie inside the file, match its shape times the dtype size, and
// not overlap another.
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace aljabr {

// dtype ids in the order of the reference's SafetensorDType enum
// (.../loader/SafetensorDType.java:35-88).
enum StDtype : int {
    kStBF16 = 0, kStF16, kStF32, kStF64, kStF8E4M3, kStF8E5M2, kStI8, kStI16, kStI32, kStI64,
    kStU8, kStU16, kStU32, kStU64, kStBool, kStCount
};

struct StTensor {
    std::string name;
    int dtype = -1;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;   // byte range in the data section
};

struct StFile {
    std::string path;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint64_t data_start = 0;
    std::vector<StTensor> tensors;
    std::vector<std::pair<std::string, std::string>> metadata;

    ~StFile();
    const StTensor *find(const std::string &name) const;
    const uint8_t *data(const StTensor &t) const { return map + data_start + t.begin; }
};

int st_dtype_bytes(int dtype);

// Opens and parses `path`; ALJABR_ROCM_OK, or an error status with the
// message set (missing file, malformed header, bad offsets).
int st_open(const char *path, StFile **out);

}  // namespace aljabr
