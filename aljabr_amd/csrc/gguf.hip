// gguf.hip - GGUF reader (host code): maps a file read-only, parses the
// header, metadata and tensor table, and exposes them through the
// aljabr_rocm_gguf_* entry points. The Llama session built from a file is in
// llama.hip (aljabr_rocm_llama_create_gguf).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <new>

#include "gguf.hpp"
#include "internal.hpp"

namespace aljabr {

GgufFile::~GgufFile() {
    if (map) munmap(const_cast<uint8_t *>(map), size);
}

const GgufValue *GgufFile::find(const std::string &key) const {
    for (const auto &kv : meta)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

const GgufTensor *GgufFile::tensor(const std::string &name) const {
    for (const auto &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

int64_t ggml_type_bytes(int type, int64_t n) {
    // (block elements, block bytes) of the ggml types (GgmlType ids).
    int be = 0, bb = 0;
    switch (type) {
    case 0: be = 1; bb = 4; break;        // F32
    case 1: be = 1; bb = 2; break;        // F16
    case 2: be = 32; bb = 18; break;      // Q4_0
    case 3: be = 32; bb = 20; break;      // Q4_1
    case 6: be = 32; bb = 22; break;      // Q5_0
    case 7: be = 32; bb = 24; break;      // Q5_1
    case 8: be = 32; bb = 34; break;      // Q8_0
    case 9: be = 32; bb = 36; break;      // Q8_1
    case 10: be = 256; bb = 84; break;    // Q2_K
    case 11: be = 256; bb = 110; break;   // Q3_K
    case 12: be = 256; bb = 144; break;   // Q4_K
    case 13: be = 256; bb = 176; break;   // Q5_K
    case 14: be = 256; bb = 210; break;   // Q6_K
    case 15: be = 256; bb = 292; break;   // Q8_K
    case 20: be = 32; bb = 18; break;     // IQ4_NL
    case 23: be = 256; bb = 136; break;   // IQ4_XS
    case 24: be = 1; bb = 1; break;       // I8
    case 25: be = 1; bb = 2; break;       // I16
    case 26: be = 1; bb = 4; break;       // I32
    case 27: be = 1; bb = 8; break;       // I64
    case 28: be = 1; bb = 8; break;       // F64
    case 30: be = 1; bb = 2; break;       // BF16
    default: return -1;
    }
    if (n < 0 || n % be != 0) return -1;
    return n / be * bb;
}

namespace {

// Little-endian reader over [p, end); any read past the end sets `bad`.
struct Cursor {
    const uint8_t *base, *p, *end;
    bool bad = false;

    template <class V>
    V get() {
        V v{};
        if (static_cast<size_t>(end - p) < sizeof(V)) {
            bad = true;
            p = end;
            return v;
        }
        std::memcpy(&v, p, sizeof(V));
        p += sizeof(V);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (bad || n > static_cast<uint64_t>(end - p)) {
            bad = true;
            p = end;
            return std::string();
        }
        std::string s(reinterpret_cast<const char *>(p), static_cast<size_t>(n));
        p += n;
        return s;
    }
    bool skip(uint64_t n) {
        if (n > static_cast<uint64_t>(end - p)) {
            bad = true;
            p = end;
            return false;
        }
        p += n;
        return true;
    }
    uint64_t pos() const { return static_cast<uint64_t>(p - base); }
};

bool read_scalar(Cursor &c, int type, GgufValue &v) {
    v.type = type;
    switch (type) {
    case 0: v.i = c.get<uint8_t>(); break;
    case 1: v.i = c.get<int8_t>(); break;
    case 2: v.i = c.get<uint16_t>(); break;
    case 3: v.i = c.get<int16_t>(); break;
    case 4: v.i = c.get<uint32_t>(); break;
    case 5: v.i = c.get<int32_t>(); break;
    case 6: v.f = c.get<float>(); break;
    case 7: v.i = c.get<uint8_t>() != 0; break;
    case 8: v.s = c.str(); break;
    case 10: v.i = static_cast<int64_t>(c.get<uint64_t>()); break;
    case 11: v.i = c.get<int64_t>(); break;
    case 12: v.f = c.get<double>(); break;
    default: return false;
    }
    return !c.bad;
}

bool read_value(Cursor &c, int type, GgufValue &v) {
    if (type != 9) return read_scalar(c, type, v);
    v.type = 9;
    v.array_type = static_cast<int>(c.get<uint32_t>());
    v.array_len = c.get<uint64_t>();
    if (c.bad || v.array_type == 9) return false;      // nested arrays are not part of GGUF
    static const int fixed[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (v.array_type < 0 || v.array_type > 12) return false;
    if (v.array_type == 8) {
        for (uint64_t i = 0; i < v.array_len && !c.bad; ++i) c.skip(c.get<uint64_t>());
        return !c.bad;
    }
    const uint64_t w = static_cast<uint64_t>(fixed[v.array_type]);
    if (v.array_len > (static_cast<uint64_t>(c.end - c.p)) / w) return false;
    return c.skip(v.array_len * w);
}

}  // namespace

int gguf_open(const char *path, GgufFile **out) {
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: cannot open %s: %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: %s is not a GGUF file (too short)", path);
    }
    void *map = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail(ALJABR_ROCM_ERR_BUFFER, "gguf: mmap %s: %s", path, std::strerror(errno));
    GgufFile *g = new (std::nothrow) GgufFile();
    if (!g) {
        munmap(map, static_cast<size_t>(st.st_size));
        return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    }
    g->path = path;
    g->map = static_cast<const uint8_t *>(map);
    g->size = static_cast<size_t>(st.st_size);
    auto bad = [&](const char *what) {
        delete g;
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: %s: %s", path, what);
    };
    Cursor c{g->map, g->map, g->map + g->size};
    if (std::memcmp(c.p, "GGUF", 4) != 0) return bad("bad magic (not a GGUF file)");
    c.p += 4;
    g->version = c.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return bad("unsupported GGUF version (2 and 3 are read)");
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (n_tensors > g->size / 8 || n_kv > g->size / 8) return bad("implausible tensor or key count");
    // The tables grow as entries are read (every entry consumes file bytes),
    // never from the counts alone; a failed host allocation is a status.
    try {
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = c.str();
        const int type = static_cast<int>(c.get<uint32_t>());
        GgufValue v;
        if (c.bad || !read_value(c, type, v)) return bad("truncated or malformed metadata");
        g->meta.emplace_back(std::move(key), std::move(v));
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensor t;
        t.name = c.str();
        t.n_dims = static_cast<int>(c.get<uint32_t>());
        if (c.bad || t.n_dims < 1 || t.n_dims > 4) return bad("tensor with 0 or more than 4 dimensions");
        int64_t n = 1;
        for (int d = 0; d < t.n_dims; ++d) {
            t.dims[d] = static_cast<int64_t>(c.get<uint64_t>());
            if (t.dims[d] < 1 || t.dims[d] > (int64_t(1) << 40) || n > (int64_t(1) << 50) / t.dims[d])
                return bad("tensor dimension out of range");
            n *= t.dims[d];
        }
        t.type = static_cast<int>(c.get<uint32_t>());
        t.offset = c.get<uint64_t>();
        if (c.bad) return bad("truncated tensor table");
        const int64_t bytes = ggml_type_bytes(t.type, n);
        if (bytes < 0) {
            delete g;
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "gguf: %s: tensor %s has unsupported type %d or a partial block",
                        path, t.name.c_str(), t.type);
        }
        t.bytes = static_cast<uint64_t>(bytes);
        g->tensors.push_back(std::move(t));
    }
    } catch (const std::bad_alloc &) {
        delete g;
        return fail(ALJABR_ROCM_ERR_BUFFER, "gguf: %s: out of host memory reading the header", path);
    }
    uint64_t align = 32;
    if (const GgufValue *a = g->find("general.alignment"))
        if (a->type != 8 && a->type != 9 && a->i > 0) align = static_cast<uint64_t>(a->i);
    if (align > g->size) return bad("general.alignment larger than the file");
    g->data_start = (c.pos() + align - 1) / align * align;
    if (g->data_start > g->size) return bad("tensor data starts past the end of the file");
    // data_start <= size, so size - data_start cannot wrap, and neither can
    // the subtraction below once offset <= size - data_start.
    for (const auto &t : g->tensors)
        if (t.offset % align != 0 || t.offset > g->size - g->data_start ||
            t.bytes > g->size - g->data_start - t.offset)
            return bad("tensor data outside the file or misaligned");
    *out = g;
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr

using namespace aljabr;

struct aljabr_rocm_gguf {
    GgufFile *f = nullptr;
    ~aljabr_rocm_gguf() { delete f; }
};

extern "C" {

int aljabr_rocm_gguf_open(const char *path, aljabr_rocm_gguf **out) {
    ALJ_REQUIRE(path && out, "path and out must be non-null");
    *out = nullptr;
    aljabr_rocm_gguf *h = new (std::nothrow) aljabr_rocm_gguf();
    if (!h) return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    const int rc = gguf_open(path, &h->f);
    if (rc != ALJABR_ROCM_OK) {
        delete h;
        return rc;
    }
    *out = h;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_close(aljabr_rocm_gguf *g) {
    delete g;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_tensor_count(const aljabr_rocm_gguf *g, int64_t *n) {
    ALJ_REQUIRE(g && n, "file and out must be non-null");
    *n = static_cast<int64_t>(g->f->tensors.size());
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_find_tensor(const aljabr_rocm_gguf *g, const char *name, int64_t *index) {
    ALJ_REQUIRE(g && name && index, "file, name and out must be non-null");
    for (size_t i = 0; i < g->f->tensors.size(); ++i)
        if (g->f->tensors[i].name == name) {
            *index = static_cast<int64_t>(i);
            return ALJABR_ROCM_OK;
        }
    return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: no tensor %s", name);
}

int aljabr_rocm_gguf_tensor_info(const aljabr_rocm_gguf *g, int64_t index, char *name, int name_cap, int32_t *type,
                                 int32_t *n_dims, int64_t *dims, uint64_t *offset, uint64_t *bytes) {
    ALJ_REQUIRE(g, "file must be non-null");
    ALJ_REQUIRE(index >= 0 && index < static_cast<int64_t>(g->f->tensors.size()), "tensor index %lld out of range",
                static_cast<long long>(index));
    const GgufTensor &t = g->f->tensors[static_cast<size_t>(index)];
    if (name && name_cap > 0) {
        std::strncpy(name, t.name.c_str(), static_cast<size_t>(name_cap) - 1);
        name[name_cap - 1] = '\0';
    }
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (offset) *offset = g->f->data_start + t.offset;
    if (bytes) *bytes = t.bytes;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_tensor_data(const aljabr_rocm_gguf *g, int64_t index, const void **host_data) {
    ALJ_REQUIRE(g && host_data, "file and out must be non-null");
    ALJ_REQUIRE(index >= 0 && index < static_cast<int64_t>(g->f->tensors.size()), "tensor index %lld out of range",
                static_cast<long long>(index));
    *host_data = g->f->data(g->f->tensors[static_cast<size_t>(index)]);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_meta_int(const aljabr_rocm_gguf *g, const char *key, int64_t *value) {
    ALJ_REQUIRE(g && key && value, "file, key and out must be non-null");
    const GgufValue *v = g->f->find(key);
    if (!v) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: no key %s", key);
    if (v->type == 9) {                          // arrays report their length
        *value = static_cast<int64_t>(v->array_len);
        return ALJABR_ROCM_OK;
    }
    ALJ_REQUIRE(v->type != 6 && v->type != 12 && v->type != 8, "gguf: key %s is not an integer", key);
    *value = v->i;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_meta_float(const aljabr_rocm_gguf *g, const char *key, double *value) {
    ALJ_REQUIRE(g && key && value, "file, key and out must be non-null");
    const GgufValue *v = g->f->find(key);
    if (!v) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: no key %s", key);
    ALJ_REQUIRE(v->type != 8 && v->type != 9, "gguf: key %s is not a number", key);
    *value = (v->type == 6 || v->type == 12) ? v->f : static_cast<double>(v->i);
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_gguf_meta_string(const aljabr_rocm_gguf *g, const char *key, char *buf, int cap) {
    ALJ_REQUIRE(g && key && buf && cap > 0, "file, key and a buffer are required");
    const GgufValue *v = g->f->find(key);
    if (!v) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: no key %s", key);
    ALJ_REQUIRE(v->type == 8, "gguf: key %s is not a string", key);
    std::strncpy(buf, v->s.c_str(), static_cast<size_t>(cap) - 1);
    buf[cap - 1] = '\0';
    return ALJABR_ROCM_OK;
}

}  // extern "C"
