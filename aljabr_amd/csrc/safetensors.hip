// safetensors.hip - safetensors reader (host code): maps a file read-only,
// parses the JSON header with a small strict parser, validates every tensor's
// byte range, and exposes the result through aljabr_rocm_safetensors_*;
// aljabr_rocm_safetensors_upload_nf4 moves one NF4 weight (codes + scales)
// to device memory in the layout the NF4 kernels read. The Llama session
// built from a file is in llama.hip (aljabr_rocm_llama_create_safetensors).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <new>
#include <unordered_set>

#include "internal.hpp"
#include "safetensors.hpp"

namespace aljabr {

namespace {

constexpr uint64_t kMaxHeader = 100ull << 20;   // SafetensorHeaderParser.java:62
constexpr int kMaxRank = 8;

const char *const kDtypeNames[kStCount] = {"BF16", "F16", "F32", "F64", "F8_E4M3", "F8_E5M2", "I8", "I16",
                                           "I32", "I64", "U8", "U16", "U32", "U64", "BOOL"};
const int kDtypeBytes[kStCount] = {2, 2, 4, 8, 1, 1, 1, 2, 4, 8, 1, 2, 4, 8, 1};

// Minimal strict JSON reader over the header bytes: objects, arrays,
// strings (with escapes), integers, true/false/null. Fails on anything else.
struct Json {
    const char *p, *end;
    bool ok = true;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool string(std::string &out) {
        ws();
        if (p >= end || *p != '"') return ok = false;
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (static_cast<unsigned char>(c) < 0x20) return ok = false;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p >= end) return ok = false;
            c = *p++;
            switch (c) {
            case '"': case '\\': case '/': out.push_back(c); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                if (end - p < 4) return ok = false;
                unsigned v = 0;
                for (int i = 0; i < 4; ++i) {
                    const char h = *p++;
                    v <<= 4;
                    if (h >= '0' && h <= '9') v |= static_cast<unsigned>(h - '0');
                    else if (h >= 'a' && h <= 'f') v |= static_cast<unsigned>(h - 'a' + 10);
                    else if (h >= 'A' && h <= 'F') v |= static_cast<unsigned>(h - 'A' + 10);
                    else return ok = false;
                }
                // UTF-8 of a BMP code point (surrogate pairs are kept as two units).
                if (v < 0x80) {
                    out.push_back(static_cast<char>(v));
                } else if (v < 0x800) {
                    out.push_back(static_cast<char>(0xC0 | (v >> 6)));
                    out.push_back(static_cast<char>(0x80 | (v & 0x3F)));
                } else {
                    out.push_back(static_cast<char>(0xE0 | (v >> 12)));
                    out.push_back(static_cast<char>(0x80 | ((v >> 6) & 0x3F)));
                    out.push_back(static_cast<char>(0x80 | (v & 0x3F)));
                }
                break;
            }
            default: return ok = false;
            }
        }
        if (p >= end) return ok = false;
        ++p;
        return true;
    }
    bool integer(int64_t &out) {
        ws();
        const char *s = p;
        if (p < end && *p == '-') ++p;
        if (p >= end || *p < '0' || *p > '9') return ok = false;
        __int128 v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            v = v * 10 + (*p++ - '0');
            if (v > (static_cast<__int128>(1) << 62)) return ok = false;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return ok = false;   // integers only
        out = static_cast<int64_t>(*s == '-' ? -v : v);
        return true;
    }
    // Skips any value (for keys the loader does not read).
    bool skip(int depth = 0) {
        ws();
        if (p >= end || depth > 64) return ok = false;
        if (*p == '"') {
            std::string s;
            return string(s);
        }
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            ++p;
            if (eat(close)) return true;
            do {
                if (obj) {
                    std::string k;
                    if (!string(k) || !eat(':')) return ok = false;
                }
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(close) || (ok = false);
        }
        for (const char *lit : {"true", "false", "null"}) {
            const size_t n = std::strlen(lit);
            if (static_cast<size_t>(end - p) >= n && std::memcmp(p, lit, n) == 0) {
                p += n;
                return true;
            }
        }
        int64_t v;
        return integer(v) || (ok = false);
    }
};

int dtype_id(const std::string &s) {
    for (int i = 0; i < kStCount; ++i)
        if (s == kDtypeNames[i]) return i;
    return -1;
}

}  // namespace

StFile::~StFile() {
    if (map) munmap(const_cast<uint8_t *>(map), size);
}

const StTensor *StFile::find(const std::string &name) const {
    for (const StTensor &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

int st_dtype_bytes(int dtype) { return dtype >= 0 && dtype < kStCount ? kDtypeBytes[dtype] : -1; }

int st_open(const char *path, StFile **out) {
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: cannot open %s: %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 10) {
        close(fd);
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s is too short", path);
    }
    void *map = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail(ALJABR_ROCM_ERR_BUFFER, "safetensors: mmap %s: %s", path, std::strerror(errno));
    StFile *f = new (std::nothrow) StFile();
    if (!f) {
        munmap(map, static_cast<size_t>(st.st_size));
        return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    }
    f->path = path;
    f->map = static_cast<const uint8_t *>(map);
    f->size = static_cast<size_t>(st.st_size);
    auto bad = [&](const char *why) {
        delete f;
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: %s", path, why);
    };
    uint64_t n = 0;
    std::memcpy(&n, f->map, 8);   // little-endian host
    if (n < 2 || n > kMaxHeader || n > f->size - 8) return bad("header length out of range");
    f->data_start = 8 + n;
    const uint64_t data_bytes = f->size - f->data_start;
    Json js{reinterpret_cast<const char *>(f->map) + 8, reinterpret_cast<const char *>(f->map) + 8 + n};
    if (!js.eat('{')) return bad("header is not a JSON object");
    if (!js.eat('}')) {
        do {
            std::string key;
            if (!js.string(key) || !js.eat(':')) return bad("malformed header");
            if (key == "__metadata__") {
                if (!js.eat('{')) return bad("__metadata__ is not an object");
                if (!js.eat('}')) {
                    do {
                        std::string k, v;
                        if (!js.string(k) || !js.eat(':') || !js.string(v)) return bad("__metadata__ values must be strings");
                        f->metadata.emplace_back(k, v);
                    } while (js.eat(','));
                    if (!js.eat('}')) return bad("malformed __metadata__");
                }
                continue;
            }
            StTensor t;
            t.name = key;
            bool have_dtype = false, have_shape = false, have_off = false;
            if (!js.eat('{')) return bad("tensor entry is not an object");
            if (!js.eat('}')) {
                do {
                    std::string fk;
                    if (!js.string(fk) || !js.eat(':')) return bad("malformed tensor entry");
                    if (fk == "dtype") {
                        std::string d;
                        if (!js.string(d)) return bad("dtype is not a string");
                        t.dtype = dtype_id(d);
                        if (t.dtype < 0) return bad("unknown dtype");
                        have_dtype = true;
                    } else if (fk == "shape") {
                        if (!js.eat('[')) return bad("shape is not an array");
                        if (!js.eat(']')) {
                            do {
                                int64_t v;
                                if (!js.integer(v) || v < 0) return bad("shape entries must be non-negative integers");
                                t.shape.push_back(v);
                            } while (js.eat(','));
                            if (!js.eat(']')) return bad("malformed shape");
                        }
                        if (t.shape.size() > kMaxRank) return bad("tensor rank above 8");
                        have_shape = true;
                    } else if (fk == "data_offsets") {
                        int64_t a, b;
                        if (!js.eat('[') || !js.integer(a) || !js.eat(',') || !js.integer(b) || !js.eat(']'))
                            return bad("data_offsets must be [begin, end]");
                        if (a < 0 || b < a) return bad("data_offsets out of order");
                        t.begin = static_cast<uint64_t>(a);
                        t.end = static_cast<uint64_t>(b);
                        have_off = true;
                    } else if (!js.skip()) {
                        return bad("malformed tensor entry");
                    }
                } while (js.eat(','));
                if (!js.eat('}')) return bad("malformed tensor entry");
            }
            if (!have_dtype || !have_shape || !have_off) return bad("tensor entry lacks dtype, shape or data_offsets");
            if (t.end > data_bytes) return bad("tensor data past the end of the file");
            __int128 numel = 1;
            for (int64_t d : t.shape) {
                numel *= d;
                if (numel > (static_cast<__int128>(1) << 60)) return bad("tensor too large");
            }
            if (static_cast<__int128>(t.end - t.begin) != numel * kDtypeBytes[t.dtype])
                return bad("data_offsets do not match shape and dtype");
            f->tensors.push_back(std::move(t));
        } while (js.eat(','));
        if (!js.eat('}')) return bad("malformed header");
    }
    js.ws();
    if (!js.ok || js.p != js.end) return bad("trailing bytes after the header object");
    // Ranges must not overlap (SafetensorValidator.java:112-190).
    std::vector<const StTensor *> order;
    for (const StTensor &t : f->tensors)
        if (t.end > t.begin) order.push_back(&t);
    std::sort(order.begin(), order.end(), [](const StTensor *a, const StTensor *b) { return a->begin < b->begin; });
    for (size_t i = 1; i < order.size(); ++i)
        if (order[i]->begin < order[i - 1]->end) return bad("tensor data ranges overlap");
    std::unordered_set<std::string> names;
    for (const StTensor &t : f->tensors)
        if (!names.insert(t.name).second) return bad("duplicate tensor name");
    *out = f;
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr

using namespace aljabr;

struct aljabr_rocm_safetensors {
    StFile *f = nullptr;
    ~aljabr_rocm_safetensors() { delete f; }
};

extern "C" {

int aljabr_rocm_safetensors_open(const char *path, aljabr_rocm_safetensors **out) {
    ALJ_REQUIRE(path && out, "path and out must be non-null");
    *out = nullptr;
    aljabr_rocm_safetensors *h = new (std::nothrow) aljabr_rocm_safetensors();
    if (!h) return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    const int rc = st_open(path, &h->f);
    if (rc != ALJABR_ROCM_OK) {
        delete h;
        return rc;
    }
    *out = h;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_safetensors_close(aljabr_rocm_safetensors *f) {
    delete f;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_safetensors_tensor_count(const aljabr_rocm_safetensors *f, int64_t *count) {
    ALJ_REQUIRE(f && count, "file and out must be non-null");
    *count = static_cast<int64_t>(f->f->tensors.size());
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_safetensors_find_tensor(const aljabr_rocm_safetensors *f, const char *name, int64_t *index) {
    ALJ_REQUIRE(f && name && index, "file, name and out must be non-null");
    for (size_t i = 0; i < f->f->tensors.size(); ++i)
        if (f->f->tensors[i].name == name) {
            *index = static_cast<int64_t>(i);
            return ALJABR_ROCM_OK;
        }
    *index = -1;
    return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: no tensor %s", name);
}

int aljabr_rocm_safetensors_tensor_info(const aljabr_rocm_safetensors *f, int64_t index, char *name, int name_cap,
                                        int32_t *dtype, int32_t *n_dims, int64_t *dims, uint64_t *bytes) {
    ALJ_REQUIRE(f, "file must be non-null");
    ALJ_REQUIRE(index >= 0 && index < static_cast<int64_t>(f->f->tensors.size()), "tensor index %lld out of range",
                static_cast<long long>(index));
    const StTensor &t = f->f->tensors[static_cast<size_t>(index)];
    if (name && name_cap > 0) {
        std::strncpy(name, t.name.c_str(), static_cast<size_t>(name_cap) - 1);
        name[name_cap - 1] = '\0';
    }
    if (dtype) *dtype = t.dtype;
    if (n_dims) *n_dims = static_cast<int32_t>(t.shape.size());
    if (dims)
        for (int d = 0; d < kMaxRank; ++d) dims[d] = d < static_cast<int>(t.shape.size()) ? t.shape[d] : 0;
    if (bytes) *bytes = t.end - t.begin;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_safetensors_tensor_data(const aljabr_rocm_safetensors *f, int64_t index, const void **host_data) {
    ALJ_REQUIRE(f && host_data, "file and out must be non-null");
    ALJ_REQUIRE(index >= 0 && index < static_cast<int64_t>(f->f->tensors.size()), "tensor index %lld out of range",
                static_cast<long long>(index));
    *host_data = f->f->data(f->f->tensors[static_cast<size_t>(index)]);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_safetensors_meta(const aljabr_rocm_safetensors *f, const char *key, char *value, int value_cap) {
    ALJ_REQUIRE(f && key && value && value_cap > 0, "file, key and a value buffer are required");
    for (const auto &kv : f->f->metadata)
        if (kv.first == key) {
            ALJ_REQUIRE(kv.second.size() < static_cast<size_t>(value_cap), "safetensors: value of %s needs %zu bytes",
                        key, kv.second.size() + 1);
            std::memcpy(value, kv.second.c_str(), kv.second.size() + 1);
            return ALJABR_ROCM_OK;
        }
    return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: no metadata key %s", key);
}

// AccelWeightBridge.java:184-222: "<base>.qweight" U8 [N, K/2] (two NF4
// codes a byte, high nibble first) with "<base>.scales" (one fp32 absmax per
// 128 weights) is an NF4 weight of logical shape [N, K], group size 128.
int aljabr_rocm_safetensors_upload_nf4(const aljabr_rocm_safetensors *f, const char *base_name, void **codes,
                                       void **absmax, int64_t *rows, int64_t *cols, int32_t *block_size) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(f && base_name && codes && absmax, "file, base name and outputs must be non-null");
    *codes = nullptr;
    *absmax = nullptr;
    const std::string base = base_name;
    const StTensor *q = f->f->find(base + ".qweight");
    const StTensor *sc = f->f->find(base + ".scales");
    if (!q || !sc) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s.qweight / %s.scales not found",
                               base_name, base_name);
    if (q->dtype != kStU8 || q->shape.size() != 2)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "safetensors: %s.qweight is not a 2-D U8 NF4 tensor", base_name);
    if (sc->dtype != kStF32)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "safetensors: %s.scales must be F32 (the NF4 kernels read fp32 "
                    "absmax)", base_name);
    const int64_t n = q->shape[0], k = 2 * q->shape[1];
    constexpr int64_t kGroup = 128;   // AccelWeightBridge.java:213
    if (n <= 0 || k % kGroup != 0 || static_cast<int64_t>((sc->end - sc->begin) / 4) != n * k / kGroup)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: %lld rows of %lld weights need %lld scales", base_name,
                    static_cast<long long>(n), static_cast<long long>(k), static_cast<long long>(n * k / kGroup));
    void *c = nullptr, *a = nullptr;
    hipError_t e = hipMalloc(&c, q->end - q->begin);
    if (e == hipSuccess) e = hipMalloc(&a, sc->end - sc->begin);
    if (e == hipSuccess) e = hipMemcpy(c, f->f->data(*q), q->end - q->begin, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(a, f->f->data(*sc), sc->end - sc->begin, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (c) (void)hipFree(c);
        if (a) (void)hipFree(a);
        return fail(ALJABR_ROCM_ERR_BUFFER, "safetensors: uploading %s: %s", base_name, hipGetErrorString(e));
    }
    *codes = c;
    *absmax = a;
    if (rows) *rows = n;
    if (cols) *cols = k;
    if (block_size) *block_size = static_cast<int32_t>(kGroup);
    return ALJABR_ROCM_OK;
}

}  // extern "C"
