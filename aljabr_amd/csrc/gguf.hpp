// gguf.hpp - a GGUF file mapped read-only and parsed (header, metadata,
// tensor table), the loader behind aljabr_rocm_gguf_* and
// aljabr_rocm_llama_create_gguf. Restates the format as the reference's
// parser reads it (engine/gguf/aljabr-gguf-core/.../loader/GGUFParser.java:18-63):
// "GGUF", version, tensor count, KV count (little endian, 64-bit counts),
// KV pairs (string key, value type, value), tensor infos (name, n_dims,
// dims, ggml type, offset), data at the next general.alignment (default 32)
// boundary. Every read is bounds-checked against the mapping.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace aljabr {

struct GgufValue {
    int type = -1;                 // GGUF value type (0..12); arrays: 9
    int64_t i = 0;                 // integer and bool types
    double f = 0.0;                // float32 / float64
    std::string s;                 // string
    int array_type = -1;           // arrays: element type and length
    uint64_t array_len = 0;
};

struct GgufTensor {
    std::string name;
    int n_dims = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    int type = -1;                 // ggml type id
    uint64_t offset = 0;           // from the data start
    uint64_t bytes = 0;
};

struct GgufFile {
    std::string path;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    std::vector<std::pair<std::string, GgufValue>> meta;
    std::vector<GgufTensor> tensors;

    ~GgufFile();
    const GgufValue *find(const std::string &key) const;
    const GgufTensor *tensor(const std::string &name) const;
    const uint8_t *data(const GgufTensor &t) const { return map + data_start + t.offset; }
};

// Bytes of `n` elements of ggml type `type`, or -1 for a type or element
// count the loader does not know.
int64_t ggml_type_bytes(int type, int64_t n);

// Opens and parses `path`; ALJABR_ROCM_OK, or an error status with the
// message set (missing file, malformed or truncated data, unknown types).
int gguf_open(const char *path, GgufFile **out);

}  // namespace aljabr
