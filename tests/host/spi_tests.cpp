// spi_tests.cpp - tests of the C++ Backend-SPI mirror (aljabr_amd/host) in the
// shape of the reference's own provider and backend tests: lifecycle and
// descriptor rules run anywhere; compute tests open a session on the first
// ROCm device and compare each op with the oracle (oracle/aljabr_oracle.c, a
// test-only C restatement of the reference CPU path) at relative L2 <= 1e-3.
//
//   spi_tests --list            names and kinds ("cpu" or "gpu"), one a line
//   spi_tests <name>...         run the named tests; exit status 0 = all passed
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "../../aljabr_amd/host/spi.hpp"
#include "../../oracle/aljabr_oracle.h"

using namespace aljabr::spi;

namespace {

struct Case {
    const char *kind;
    std::function<void()> fn;
};
std::map<std::string, Case> &registry() {
    static std::map<std::string, Case> r;
    return r;
}
struct Reg {
    Reg(const char *name, const char *kind, std::function<void()> fn) { registry()[name] = {kind, std::move(fn)}; }
};
#define TEST(name, kind) \
    static void name();  \
    static Reg reg_##name(#name, kind, name); \
    static void name()

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};
#define EXPECT(cond)                                                                              \
    do {                                                                                          \
        if (!(cond)) throw Failure(std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond); \
    } while (0)

template <typename E, typename F>
void expect_throws(F &&f, const char *what) {
    try {
        f();
    } catch (const E &) {
        return;
    } catch (const std::exception &e) {
        throw Failure(std::string(what) + ": threw the wrong exception: " + e.what());
    }
    throw Failure(std::string(what) + ": did not throw");
}

double rel_l2(const std::vector<float> &a, const std::vector<float> &e) {
    double num = 0, den = 0;
    for (size_t i = 0; i < a.size(); ++i) {
        const double d = static_cast<double>(a[i]) - e[i];
        num += d * d;
        den += static_cast<double>(e[i]) * e[i];
    }
    return std::sqrt(num) / (den > 0 ? std::sqrt(den) : 1.0);
}

std::vector<float> normal(uint64_t seed, size_t n, float stdev = 1.0f) {
    std::vector<float> v(n);
    orc_fill_normal(seed, 0.0f, stdev, v.data(), static_cast<int64_t>(n));
    return v;
}

// A provider initialized and a session open on rocm:0.
struct Fixture {
    std::unique_ptr<ComputeProvider> provider = make_rocm_provider();
    std::unique_ptr<ProviderSession> session;
    ComputeBackend *backend = nullptr;
    Fixture() {
        provider->initialize(ProviderContext("0.1.0", {}));
        auto devices = provider->devices();
        if (devices.empty()) throw Failure("no ROCm device");
        session = provider->openSession(devices.front());
        backend = session->computeBackends().at("rocm-default");
    }
    template <typename T>
    Tensor upload(const std::vector<T> &host, std::vector<long long> shape, DType dt) {
        TensorStorage *s = backend->allocateStorage(static_cast<long long>(host.size() * sizeof(T)));
        backend->copyFromHost(s, host.data(), static_cast<long long>(host.size() * sizeof(T)));
        return Tensor(std::move(shape), dt, s);
    }
    std::vector<float> download(const Tensor &t) {
        std::vector<float> out(static_cast<size_t>(t.numel()));
        backend->copyToHost(out.data(), t.storage(), t.numel() * 4);
        return out;
    }
};

// ---- descriptors and lifecycle (no device needed) ---------------------------------

TEST(provider_descriptor_rules, "cpu") {
    auto p = make_rocm_provider();
    EXPECT(p->descriptor().id == "andalus/rocm");
    expect_throws<IllegalArgumentException>([] { ProviderDescriptor("Bad/Id", "1", ">=0.1.0"); }, "upper-case id");
    expect_throws<IllegalArgumentException>([] { ProviderDescriptor("noslash", "1", ">=0.1.0"); }, "id without namespace");
    expect_throws<IllegalArgumentException>([] { ProviderContext("  ", {}); }, "blank aljabrVersion");
}

TEST(device_descriptor_rules, "cpu") {
    DeviceDescriptor ok("andalus/rocm", " rocm:0 ", "MI355X", DeviceKind::GPU, 100, 40, std::string("AMD"),
                        std::string("  "), std::nullopt, std::nullopt);
    EXPECT(ok.deviceId == "rocm:0");
    EXPECT(!ok.architecture.has_value());      // blank optional fields normalize to empty
    expect_throws<IllegalArgumentException>(
        [] { DeviceDescriptor("andalus/rocm", "", "x", DeviceKind::GPU, {}, {}, {}, {}, {}, {}); }, "blank deviceId");
    expect_throws<IllegalArgumentException>(
        [] { DeviceDescriptor("andalus/rocm", "rocm:0", "x", DeviceKind::GPU, -1, {}, {}, {}, {}, {}); }, "negative total");
    expect_throws<IllegalArgumentException>(
        [] { DeviceDescriptor("andalus/rocm", "rocm:0", "x", DeviceKind::GPU, 10, 11, {}, {}, {}, {}); }, "free > total");
    expect_throws<IllegalArgumentException>(
        [] { OperationSupportDescriptor("tensor.matmul", OperationSupport::DELEGATED, std::string(" ")); },
        "DELEGATED without backend");
}

TEST(provider_lifecycle, "cpu") {
    auto p = make_rocm_provider();
    expect_throws<ProviderException>([&] { p->devices(); }, "devices before initialize");
    p->initialize(ProviderContext("0.1.0", {}));
    expect_throws<ProviderException>([&] { p->initialize(ProviderContext("0.1.0", {})); }, "second initialize");
    auto devices = p->devices();                 // empty where there is no GPU
    for (const auto &d : devices) {
        EXPECT(d.providerId == "andalus/rocm");
        EXPECT(d.kind == DeviceKind::GPU);
        EXPECT(d.vendor && *d.vendor == "AMD");
    }
    p->close();
    p->close();                                  // idempotent
    expect_throws<ProviderException>([&] { p->devices(); }, "devices after close");
    expect_throws<ProviderException>([&] { p->initialize(ProviderContext("0.1.0", {})); }, "initialize after close");
}

TEST(open_session_rejects_foreign_device, "cpu") {
    auto p = make_rocm_provider();
    p->initialize(ProviderContext("0.1.0", {}));
    DeviceDescriptor cpu("andalus/cpu", "cpu:0", "host", DeviceKind::CPU, {}, {}, {}, {}, {}, {});
    expect_throws<ProviderException>([&] { p->openSession(cpu); }, "foreign provider id");
    DeviceDescriptor odd("andalus/rocm", "gpu7", "x", DeviceKind::GPU, {}, {}, {}, {}, {}, {});
    expect_throws<ProviderException>([&] { p->openSession(odd); }, "unknown device id");
}

// ---- session, backend map and support queries -------------------------------------

TEST(session_backends_and_close, "gpu") {
    Fixture f;
    auto map = f.session->computeBackends();
    EXPECT(map.size() == 1 && map.count("rocm-default"));
    EXPECT(f.backend->deviceType() == DeviceType::ROCM);
    auto s = f.session->operationSupport("tensor.matmul", {{"inputDtype", "F32"}, {"weightDtype", "NF4"}});
    EXPECT(s.support == OperationSupport::NATIVE);
    EXPECT(f.session->operationSupport("tensor.matmul", {{"inputDtype", "f32"}, {"weightDtype", "q4_k"}}).support ==
           OperationSupport::UNSUPPORTED);
    EXPECT(f.session->operationSupport("tensor.attention", {{"dtype", "f32"}}).support == OperationSupport::NATIVE);
    EXPECT(f.session->operationSupport("tensor.softmax", {}).support == OperationSupport::UNSUPPORTED);
    EXPECT(f.session->operationSupport("vendor.op", {}).support == OperationSupport::UNKNOWN);
    expect_throws<IllegalArgumentException>([&] { f.session->operationSupport("  ", {}); }, "blank operation id");
    f.session->close();
    f.session->close();
    expect_throws<IllegalStateException>([&] { f.session->computeBackends(); }, "backends after close");
    expect_throws<IllegalStateException>([&] { f.backend->allocateStorage(16); }, "backend after session close");
}

TEST(provider_close_closes_sessions, "gpu") {
    Fixture f;
    EXPECT(f.session->computeBackends().size() == 1);
    f.provider->close();
    expect_throws<IllegalStateException>([&] { f.session->computeBackends(); }, "session after provider close");
    expect_throws<IllegalStateException>([&] { f.backend->allocateStorage(16); }, "backend after provider close");
}

TEST(storage_ownership, "gpu") {
    Fixture f;
    TensorStorage *s = f.backend->allocateStorage(1024);
    EXPECT(s->sizeBytes() == 1024);
    s->retain();
    s->release();
    std::vector<float> host(256, 1.5f);
    f.backend->copyFromHost(s, host.data(), 1024);
    expect_throws<IllegalArgumentException>([&] { f.backend->copyFromHost(s, host.data(), 2048); }, "oversized copy");
    s->release();                                // final release frees the device memory
}

// ---- compute parity with the oracle -------------------------------------------------

void check_nf4(Fixture &f, int M, int N, int K) {
    auto w = normal(1000 + N + K, static_cast<size_t>(N) * K, 0.02f);
    std::vector<uint8_t> codes(static_cast<size_t>(N) * K / 2);
    std::vector<float> absmax(static_cast<size_t>(N) * K / 64);
    orc_nf4_quantize(w.data(), static_cast<int64_t>(w.size()), 64, codes.data(), absmax.data());
    auto x = normal(2000 + M, static_cast<size_t>(M) * K);
    std::vector<float> ref(static_cast<size_t>(M) * N);
    orc_nf4_matvec(codes.data(), absmax.data(), 64, x.data(), N, K, M, ref.data(), orc_max_threads());
    Tensor b = f.upload(codes, {N, K}, DType::NF4);
    TensorStorage *sc = f.backend->allocateStorage(static_cast<long long>(absmax.size() * 4));
    f.backend->copyFromHost(sc, absmax.data(), static_cast<long long>(absmax.size() * 4));
    Tensor bw({N, K}, DType::NF4, b.storage(), sc, 64);
    b.storage()->retain();                       // bw owns its own reference
    Tensor a = f.upload(x, {M, K}, DType::F32);
    Tensor y = f.backend->matmul(a, bw);
    EXPECT(y.shape() == (std::vector<long long>{M, N}));
    EXPECT(rel_l2(f.download(y), ref) <= 1e-3);
}

TEST(matmul_nf4_matches_oracle, "gpu") {
    Fixture f;
    check_nf4(f, 1, 4096, 4096);                 // batch-1 rows kernel
    check_nf4(f, 3, 300, 1024);                  // small-M on the matrix cores
    check_nf4(f, 1, 96, 2080);                   // generic path
}

TEST(matmul_gguf_matches_oracle, "gpu") {
    Fixture f;
    const int N = 333, K = 2048, M = 2;
    auto w = normal(3000, static_cast<size_t>(N) * K, 0.02f);
    auto x = normal(3001, static_cast<size_t>(M) * K);
    for (DType dt : {DType::Q4_0, DType::Q8_0}) {
        const size_t bytes = static_cast<size_t>(N) * K / 32 * (dt == DType::Q4_0 ? 18 : 34);
        std::vector<uint8_t> enc(bytes);
        std::vector<float> ref(static_cast<size_t>(M) * N);
        if (dt == DType::Q4_0) {
            orc_q4_0_quantize(w.data(), static_cast<int64_t>(w.size()), enc.data());
            orc_q4_0_matvec(enc.data(), x.data(), N, K, M, ref.data(), orc_max_threads());
        } else {
            orc_q8_0_quantize(w.data(), static_cast<int64_t>(w.size()), enc.data());
            orc_q8_0_matvec(enc.data(), x.data(), N, K, M, ref.data(), orc_max_threads());
        }
        Tensor b = f.upload(enc, {N, K}, dt);
        Tensor a = f.upload(x, {M, K}, DType::F32);
        Tensor y = f.backend->matmul(a, b);
        EXPECT(rel_l2(f.download(y), ref) <= 1e-3);
    }
    Tensor a = f.upload(x, {M, K}, DType::F32);
    Tensor bad = f.upload(std::vector<float>(16), {4, 4}, DType::F32);
    expect_throws<IllegalArgumentException>([&] { f.backend->matmul(a, bad); }, "inner dimension mismatch");
}

TEST(attention_gqa_matches_oracle, "gpu") {
    Fixture f;
    const long long B = 2, Hq = 8, Hkv = 2, Sq = 3, Sk = 77, D = 64;
    auto q = normal(4000, B * Hq * Sq * D), k = normal(4001, B * Hkv * Sk * D), v = normal(4002, B * Hkv * Sk * D);
    std::vector<float> ref(static_cast<size_t>(B * Hq * Sq * D));
    EXPECT(orc_attention_gqa(q.data(), k.data(), v.data(), nullptr, B, Hq, Hkv, Sq, Sk, D, 1, ref.data(),
                             orc_max_threads()) == 0);
    Tensor Q = f.upload(q, {B, Hq, Sq, D}, DType::F32);
    Tensor K = f.upload(k, {B, Hkv, Sk, D}, DType::F32);
    Tensor V = f.upload(v, {B, Hkv, Sk, D}, DType::F32);
    Tensor out = f.backend->attentionGqa(Q, K, V, nullptr, true);
    EXPECT(rel_l2(f.download(out), ref) <= 1e-3);

    Tensor Kbad = f.upload(k, {B, 3, Sk * 2 / 3 + 1, D}, DType::F32);
    expect_throws<IllegalArgumentException>([&] { f.backend->attentionGqa(Q, Kbad, Kbad, nullptr, true); },
                                            "Hq not divisible by Hkv");
    std::vector<float> nanmask(static_cast<size_t>(Sq * Sk), 0.0f);
    nanmask[5] = std::nanf("");
    Tensor M = f.upload(nanmask, {Sq, Sk}, DType::F32);
    expect_throws<IllegalArgumentException>([&] { f.backend->attentionGqa(Q, K, V, &M, true); }, "NaN mask");
    Tensor Mshape = f.upload(nanmask, {Sk, Sq}, DType::F32);
    expect_throws<IllegalArgumentException>([&] { f.backend->attentionGqa(Q, K, V, &Mshape, true); }, "mask shape");
}

TEST(rmsnorm_rope_add_match_oracle, "gpu") {
    Fixture f;
    const int rows = 5, H = 4096;
    auto x = normal(5000, static_cast<size_t>(rows) * H), w = normal(5001, H);
    std::vector<float> ref(x.size());
    for (int r = 0; r < rows; ++r) orc_rmsnorm(x.data() + r * H, w.data(), ref.data() + r * H, H, 1e-5f);
    Tensor X = f.upload(x, {rows, H}, DType::F32), W = f.upload(w, {H}, DType::F32);
    EXPECT(rel_l2(f.download(f.backend->rmsNorm(X, W, 1e-5f)), ref) <= 1e-3);
    expect_throws<IllegalArgumentException>([&] { f.backend->rmsNorm(X, W, -1.0f); }, "negative epsilon");

    const long long B = 1, Hh = 4, S = 6, D = 128;
    auto t = normal(5002, B * Hh * S * D);
    std::vector<float> rref = t;
    for (long long h = 0; h < Hh; ++h)
        for (long long s = 0; s < S; ++s) orc_rope(rref.data() + (h * S + s) * D, 1, D, static_cast<int32_t>(7 + s), 500000.0f);
    Tensor T = f.upload(t, {B, Hh, S, D}, DType::F32);
    EXPECT(rel_l2(f.download(f.backend->applyRoPE(T, 7, 500000.0f, true)), rref) <= 1e-3);
    expect_throws<UnsupportedOperationException>([&] { f.backend->applyRoPE(T, 7, 500000.0f, false); }, "interleaved RoPE");
    expect_throws<IllegalArgumentException>([&] { f.backend->applyRoPE(T, 0, 1.0f, true); }, "freqBase <= 1");

    auto a = normal(5003, 1000), b = normal(5004, 1000);
    std::vector<float> sum(1000), sw(1000);
    for (int i = 0; i < 1000; ++i) sum[i] = a[i] + b[i];
    orc_swiglu(a.data(), b.data(), sw.data(), 1000);
    Tensor A = f.upload(a, {1000}, DType::F32), Bt = f.upload(b, {1000}, DType::F32);
    EXPECT(rel_l2(f.download(f.backend->add(A, Bt)), sum) == 0.0);
    EXPECT(rel_l2(f.download(f.backend->siluMul(A, Bt)), sw) <= 1e-3);
}

}  // namespace

int main(int argc, char **argv) {
    if (argc >= 2 && std::strcmp(argv[1], "--list") == 0) {
        for (const auto &kv : registry()) std::printf("%s %s\n", kv.first.c_str(), kv.second.kind);
        return 0;
    }
    int failed = 0;
    for (int i = 1; i < argc; ++i) {
        auto it = registry().find(argv[i]);
        if (it == registry().end()) {
            std::printf("UNKNOWN %s\n", argv[i]);
            ++failed;
            continue;
        }
        std::printf("RUN %s\n", argv[i]);
        std::fflush(stdout);
        try {
            it->second.fn();
            std::printf("PASS %s\n", argv[i]);
        } catch (const std::exception &e) {
            std::printf("FAIL %s: %s\n", argv[i], e.what());
            ++failed;
        }
        std::fflush(stdout);
    }
    return failed ? 1 : 0;
}
