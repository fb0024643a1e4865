// host_test.cpp - the reference's Go kernel and cgo tests, restated in C++
// over the C++ mirror of its bindings (neurogrid_amd/host/neurogrid_gpu.hpp),
// so that they drive libgpu_engine.so through the same wrapper calls, shape
// rules and error text as the Go host does.
//
// Sources: tests/kernels_test.go:19-274 (RMSNorm, SiLU, RoPE, Add),
// tests/quantize_test.go:20-280, tests/matmul_test.go:20-260 (GEMMFP16,
// GEMMINT8, GEMMTranspose), tests/cgo_test.go:16-313 (init/shutdown, error
// handling, call overhead, concurrent calls), tests/golden_test.go:24-201
// (RMSNorm and SiLU golden vectors) and tests/e2e/real_inference_test.go:
// 218-279 (embedding lookup). The Go suites
// draw from math/rand seed 42, which is not reproduced here; a seeded
// std::mt19937 stream serves these tolerance checks equally.
//
// Usage: host_test [--list] [--golden DIR] [name...]. Runs every test (or
// the named ones) in order, prints RUN / PASS / FAIL lines, and exits with the
// number of failures. --list prints the names and touches no GPU.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include <unistd.h>

#include "neurogrid_gpu.hpp"

namespace ng = neurogrid;

namespace {

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define CHECK(cond, ...)                                                              \
    do {                                                                              \
        if (!(cond)) {                                                                \
            char msg_[512];                                                           \
            std::snprintf(msg_, sizeof(msg_), __VA_ARGS__);                           \
            throw Failure(std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " + msg_); \
        }                                                                             \
    } while (0)

void NoError(const ng::Error& e, const char* what) {
    if (e) throw Failure(std::string(what) + ": " + e.message());
}

void WantError(const ng::Error& e, const char* substring, const char* what) {
    if (!e) throw Failure(std::string(what) + ": expected an error containing \"" + substring + "\", got nil");
    if (e.message().find(substring) == std::string::npos)
        throw Failure(std::string(what) + ": error \"" + e.message() + "\" does not contain \"" + substring + "\"");
}

// A tensor freed when it goes out of scope (the Go tests' `defer FreeTensor`).
struct Owned {
    ng::Tensor t;
    Owned(std::vector<int64_t> shape, ng::Dtype d) : t(ng::NewTensor(std::move(shape), d)) {
        NoError(ng::AllocateTensor(&t), "AllocateTensor");
    }
    ~Owned() { ng::FreeTensor(&t); }
    Owned(const Owned&) = delete;
    Owned& operator=(const Owned&) = delete;
    ng::Tensor* operator->() { return &t; }
    ng::Tensor* get() { return &t; }
};

std::vector<float> Uniform(std::mt19937& rng, size_t n) {  // rng.Float32()*2 - 1
    std::uniform_real_distribution<float> u(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto& x : v) x = u(rng) * 2.0f - 1.0f;
    return v;
}

// x rounded to the nearest fp16 value, ties to even, straight from double
// (one rounding). In the normal range the spacing of fp16 values around x is
// 2^(e-10) for 2^e <= |x| < 2^(e+1); below 2^-14 it is 2^-24. Dividing by a
// power of two is exact, so nearbyint under the default rounding mode rounds
// the scaled value to an integer with ties to even.
double RoundToHalf(double x) {
    if (x == 0.0 || std::isnan(x)) return x;
    int e = std::ilogb(x);
    if (e < -14) e = -14;
    const double ulp = std::ldexp(1.0, e - 10);
    const double r = std::nearbyint(x / ulp) * ulp;
    if (std::fabs(r) > 65504.0) return std::copysign(INFINITY, x);
    return r;
}

std::vector<float> CpuMatmul(const std::vector<float>& a, const std::vector<float>& b, int M, int K, int N) {
    std::vector<float> c(static_cast<size_t>(M) * N, 0.0f);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float s = 0.0f;
            for (int k = 0; k < K; ++k) s += a[static_cast<size_t>(i) * K + k] * b[static_cast<size_t>(k) * N + j];
            c[static_cast<size_t>(i) * N + j] = s;
        }
    return c;
}

// The reference's golden vectors (written by its scripts/generate_golden.py,
// committed under tests/golden/reference_kernels/ as raw little-endian fp32),
// found relative to this program (neurogrid_amd/lib/host_test) or given with
// --golden DIR.
std::string g_golden_dir;

std::vector<float> LoadGolden(const char* name) {
    const std::string path = g_golden_dir + "/" + name;
    FILE* f = std::fopen(path.c_str(), "rb");
    CHECK(f != nullptr, "cannot open %s", path.c_str());
    std::vector<float> v;
    float x;
    while (std::fread(&x, sizeof(float), 1, f) == 1) v.push_back(x);
    std::fclose(f);
    CHECK(!v.empty(), "%s is empty", path.c_str());
    return v;
}

// Max, mean and count above `tol` of |got - want|.
struct DiffStats {
    double max = 0, mean = 0;
    size_t over = 0;
};
DiffStats Diff(const std::vector<float>& got, const std::vector<float>& want, double tol) {
    DiffStats d;
    for (size_t i = 0; i < want.size(); ++i) {
        const double e = std::fabs(static_cast<double>(got[i]) - want[i]);
        d.max = std::max(d.max, e);
        d.mean += e;
        d.over += e > tol;
    }
    d.mean /= static_cast<double>(want.size());
    return d;
}

// ------------------------------------------------------------------ tests

// cgo_test.go:16-34 runs init / info / shutdown / re-init; the shutdown half
// resets the device and is TestCGOInitShutdown at the end of the list.
void TestDeviceInfo() {
    ng::DeviceInfo info;
    NoError(ng::GetDeviceInfo(&info), "GetDeviceInfo");
    std::printf("  GPU: %s, gfx%d.%d, memory %llu MiB\n", info.Name.c_str(), info.Major, info.Minor,
                static_cast<unsigned long long>(info.TotalMemory >> 20));
    CHECK(info.TotalMemory > 0 && info.Major >= 9, "device info: major %d, memory %llu", info.Major,
          static_cast<unsigned long long>(info.TotalMemory));
    int count = 0;
    NoError(ng::GetDeviceCount(&count), "GetDeviceCount");
    CHECK(count >= 1 && ng::HasCUDA(), "device count %d", count);
    uint64_t used = 0;
    NoError(ng::GetMemoryUsed(&used), "GetMemoryUsed");
    CHECK(used > 0, "memory used %llu", static_cast<unsigned long long>(used));
}

// kernels_test.go:19-106: hidden 4096 (Llama-7B), eps 1e-6, input i*0.001,
// unit weight; fewer than 10 elements off by more than 0.2 % relative.
void TestRMSNorm() {
    const int H = 4096;
    const float eps = 1e-6f;
    Owned in({1, 1, H}, ng::Dtype::FP16), w({H}, ng::Dtype::FP16), out({1, 1, H}, ng::Dtype::FP16);
    std::vector<float> x(H), ones(H, 1.0f);
    for (int i = 0; i < H; ++i) x[i] = static_cast<float>(i) * 0.001f;
    NoError(ng::CopyToDevice(in.get(), x), "CopyToDevice");
    NoError(ng::CopyToDevice(w.get(), ones), "CopyToDevice");
    NoError(ng::RMSNorm(out.get(), in.get(), w.get(), eps), "RMSNorm");
    std::vector<float> res(H);
    NoError(ng::CopyToHost(res, out.get()), "CopyToHost");
    double ss = 0;
    for (float v : x) ss += static_cast<double>(v) * v;
    const double rs = 1.0 / std::sqrt(ss / H + eps);
    int bad = 0;
    for (int i = 0; i < H; ++i) {
        const double want = x[i] * rs;
        if (want != 0 && std::fabs(res[i] - want) / std::fabs(want) > 0.002) ++bad;
    }
    CHECK(bad < 10, "%d RMSNorm elements off by more than 0.2%%", bad);
}

// kernels_test.go:108-156: n 11008 (Llama-7B intermediate), x = (i - n/2)*0.01;
// the first 100 outputs within 1e-4 of x / (1 + e^-x).
void TestSiLU() {
    const int n = 11008;
    Owned in({1, 1, n}, ng::Dtype::FP16), out({1, 1, n}, ng::Dtype::FP16);
    std::vector<float> x(n);
    for (int i = 0; i < n; ++i) x[i] = static_cast<float>(i - n / 2) * 0.01f;
    NoError(ng::CopyToDevice(in.get(), x), "CopyToDevice");
    NoError(ng::SiLU(out.get(), in.get()), "SiLU");
    std::vector<float> res(n);
    NoError(ng::CopyToHost(res, out.get()), "CopyToHost");
    for (int i = 0; i < 100; ++i) {
        const double want = x[i] / (1.0 + std::exp(-static_cast<double>(x[i])));
        CHECK(std::fabs(res[i] - want) < 1e-4, "SiLU[%d] = %g, want %g", i, res[i], want);
    }
}

// kernels_test.go:158-213: [1, 4, 32, 128] of ones, positions i % 4; the
// output differs from the input. Position 0 is the identity rotation, so its
// token stays exactly 1.
void TestRoPE() {
    const std::vector<int64_t> shape{1, 4, 32, 128};
    Owned in(shape, ng::Dtype::FP16), out(shape, ng::Dtype::FP16);
    const int64_t n = in->NumElements();
    NoError(ng::CopyToDevice(in.get(), std::vector<float>(n, 1.0f)), "CopyToDevice");
    std::vector<int32_t> pos(4);
    for (int i = 0; i < 4; ++i) pos[i] = i % 4;
    NoError(ng::RoPE(out.get(), in.get(), pos, 128), "RoPE");
    std::vector<float> res(n);
    NoError(ng::CopyToHost(res, out.get()), "CopyToHost");
    bool different = false;
    for (float v : res) different |= std::fabs(v - 1.0f) > 1e-6f;
    CHECK(different, "RoPE left every value unchanged");
    for (int i = 0; i < 32 * 128; ++i) CHECK(res[i] == 1.0f, "position 0 changed element %d to %g", i, res[i]);
}

// kernels_test.go:215-274: a = i*0.001, b = (n - i)*0.001; fewer than 10
// elements off by more than 0.01.
void TestAddKernel() {
    const int n = 4096;
    Owned a({n}, ng::Dtype::FP16), b({n}, ng::Dtype::FP16), c({n}, ng::Dtype::FP16);
    std::vector<float> da(n), db(n);
    for (int i = 0; i < n; ++i) {
        da[i] = static_cast<float>(i) * 0.001f;
        db[i] = static_cast<float>(n - i) * 0.001f;
    }
    NoError(ng::CopyToDevice(a.get(), da), "CopyToDevice");
    NoError(ng::CopyToDevice(b.get(), db), "CopyToDevice");
    NoError(ng::Add(c.get(), a.get(), b.get()), "Add");
    std::vector<float> res(n);
    NoError(ng::CopyToHost(res, c.get()), "CopyToHost");
    int bad = 0;
    for (int i = 0; i < n; ++i) bad += std::fabs(res[i] - (da[i] + db[i])) > 0.01f;
    CHECK(bad < 10, "%d Add elements off by more than 0.01", bad);
}

// quantize_test.go:20-87: 4096 values U(-1, 1); scale within 0.01 of
// max|x|/127 and every reconstruction within 0.01.
void TestQuantizePerTensor() {
    const int n = 4096;
    std::mt19937 rng(42);
    const std::vector<float> data = Uniform(rng, n);
    Owned in({n}, ng::Dtype::FP16), out({n}, ng::Dtype::INT8), sc({1}, ng::Dtype::FP32);
    NoError(ng::CopyToDevice(in.get(), data), "CopyToDevice");
    NoError(ng::QuantizePerTensor(out.get(), sc.get(), in.get()), "QuantizePerTensor");
    std::vector<int8_t> q(n);
    std::vector<float> s(1);
    NoError(ng::CopyToHostINT8(q, out.get()), "CopyToHostINT8");
    NoError(ng::CopyToHost(s, sc.get()), "CopyToHost");
    float amax = 0;
    for (float v : data) amax = std::max(amax, std::fabs(v));
    CHECK(std::fabs(amax / 127.0f - s[0]) < 0.01f, "scale %g, max|x|/127 %g", s[0], amax / 127.0f);
    for (int i = 0; i < n; ++i)
        CHECK(std::fabs(data[i] - q[i] * s[0]) < 0.01f, "element %d: %g vs %d * %g", i, data[i], q[i], s[0]);
}

// quantize_test.go:89-154: 4096 codes U{-128..127}, scale 0.01; fewer than 10
// outputs off by more than 1e-3.
void TestDequantizePerTensor() {
    const int n = 4096;
    std::mt19937 rng(42);
    std::uniform_int_distribution<int> u(-128, 127);
    std::vector<int8_t> codes(n);
    for (auto& c : codes) c = static_cast<int8_t>(u(rng));
    Owned in({n}, ng::Dtype::INT8), out({n}, ng::Dtype::FP16), sc({1}, ng::Dtype::FP32);
    NoError(ng::CopyToDeviceINT8(in.get(), codes), "CopyToDeviceINT8");
    NoError(ng::CopyToDevice(sc.get(), {0.01f}), "CopyToDevice");
    NoError(ng::DequantizePerTensor(out.get(), in.get(), sc.get()), "DequantizePerTensor");
    std::vector<float> res(n);
    NoError(ng::CopyToHost(res, out.get()), "CopyToHost");
    int bad = 0;
    for (int i = 0; i < n; ++i) bad += std::fabs(res[i] - codes[i] * 0.01f) > 1e-3f;
    CHECK(bad < 10, "%d dequantized elements off by more than 1e-3", bad);
}

// quantize_test.go:156-280 (TestQuantizeWeights, TestQuantizeRoundtrip):
// [128, 64] U(-1, 1), per-column scales; max and mean reconstruction error
// under 0.01.
void TestQuantizeWeights() {
    const int K = 128, N = 64;
    std::mt19937 rng(42);
    const std::vector<float> w = Uniform(rng, static_cast<size_t>(K) * N);
    Owned in({K, N}, ng::Dtype::FP16), out({K, N}, ng::Dtype::INT8), sc({N}, ng::Dtype::FP32);
    NoError(ng::CopyToDevice(in.get(), w), "CopyToDevice");
    NoError(ng::QuantizeWeights(out.get(), sc.get(), in.get()), "QuantizeWeights");
    std::vector<int8_t> q(static_cast<size_t>(K) * N);
    std::vector<float> s(N);
    NoError(ng::CopyToHostINT8(q, out.get()), "CopyToHostINT8");
    NoError(ng::CopyToHost(s, sc.get()), "CopyToHost");
    double emax = 0, esum = 0;
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N; ++j) {
            const double e = std::fabs(q[k * N + j] * s[j] - w[k * N + j]);
            emax = std::max(emax, e);
            esum += e;
        }
    CHECK(emax < 0.01 && esum / (K * N) < 0.01, "max error %g, mean error %g", emax, esum / (K * N));
}

// The fp32 -> fp16 copy rounds to nearest even (memory.cu:145-213): every
// midpoint between adjacent finite fp16 values, both signs, plus 1000
// normal draws, round-trip to the fp16 value nearest the input.
void TestCopyFP16RoundToNearestEven() {
    std::vector<float> x;
    for (int e = -24; e < 16; ++e) {
        // fp16 values in [2^e, 2^(e+1)) are spaced max(2^(e-10), 2^-24) apart.
        const double step = std::ldexp(1.0, std::max(e - 10, -24));
        for (double v = std::ldexp(1.0, e); v < std::ldexp(1.0, e + 1) && v + step <= 65504.0; v += step) {
            x.push_back(static_cast<float>(v + step / 2));
            x.push_back(static_cast<float>(-(v + step / 2)));
        }
    }
    std::mt19937 rng(1);
    std::normal_distribution<float> g;
    for (int i = 0; i < 1000; ++i) x.push_back(g(rng));
    Owned t({static_cast<int64_t>(x.size())}, ng::Dtype::FP16);
    NoError(ng::CopyToDevice(t.get(), x), "CopyToDevice");
    std::vector<float> back(x.size());
    NoError(ng::CopyToHost(back, t.get()), "CopyToHost");
    for (size_t i = 0; i < x.size(); ++i)
        CHECK(back[i] == static_cast<float>(RoundToHalf(x[i])), "fp16(%a) came back %a, want %a", x[i], back[i],
              RoundToHalf(x[i]));
    std::printf("  %zu values round-tripped\n", x.size());
}

// real_inference_test.go:218-279: a [100, 128] fp16 table holding the byte
// pattern (i % 256); token 42's row comes back byte for byte.
void TestEmbeddingLookup() {
    const int V = 100, H = 128;
    std::vector<int8_t> table(static_cast<size_t>(V) * H * 2);
    for (size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int8_t>(i % 256);
    Owned tb({static_cast<int64_t>(table.size())}, ng::Dtype::INT8);
    Owned ids({4}, ng::Dtype::INT8);
    Owned out({2 * H}, ng::Dtype::INT8);
    NoError(ng::CopyToDeviceINT8(tb.get(), table), "CopyToDeviceINT8");
    const int32_t id = 42;
    std::vector<int8_t> idb(4);
    std::memcpy(idb.data(), &id, 4);
    NoError(ng::CopyToDeviceINT8(ids.get(), idb), "CopyToDeviceINT8");
    NoError(ng::GatherEmbeddings(out->Data, tb->Data, ids->Data, H, 1), "GatherEmbeddings");
    NoError(ng::SyncDevice(), "SyncDevice");
    std::vector<int8_t> got(2 * H);
    NoError(ng::CopyToHostINT8(got, out.get()), "CopyToHostINT8");
    const size_t off = static_cast<size_t>(id) * H * 2;
    for (int i = 0; i < 2 * H; ++i)
        CHECK(static_cast<uint8_t>(got[i]) == (off + i) % 256, "byte %d: %d, want %zu", i,
              static_cast<uint8_t>(got[i]), (off + i) % 256);
}

// golden_test.go:24-117: RMSNorm of the golden [1, 1, 4096] input with eps
// 1e-6 against the golden output: max |d| < 5e-3, mean < 1e-4, fewer than 1%
// of elements off by more than 1e-3.
void TestRMSNormGolden() {
    const std::vector<float> x = LoadGolden("rmsnorm_input.bin"), w = LoadGolden("rmsnorm_weight.bin"),
                             want = LoadGolden("rmsnorm_output.bin");
    const int64_t H = static_cast<int64_t>(w.size());
    CHECK(x.size() == w.size() && want.size() == w.size(), "golden sizes %zu %zu %zu", x.size(), w.size(),
          want.size());
    Owned in({1, 1, H}, ng::Dtype::FP16), wt({H}, ng::Dtype::FP16), out({1, 1, H}, ng::Dtype::FP16);
    NoError(ng::CopyToDevice(in.get(), x), "CopyToDevice");
    NoError(ng::CopyToDevice(wt.get(), w), "CopyToDevice");
    NoError(ng::RMSNorm(out.get(), in.get(), wt.get(), 1e-6f), "RMSNorm");
    std::vector<float> got(H);
    NoError(ng::CopyToHost(got, out.get()), "CopyToHost");
    const DiffStats d = Diff(got, want, 1e-3);
    std::printf("  max_diff %.3e, avg_diff %.3e, errors %zu/%lld\n", d.max, d.mean, d.over,
                static_cast<long long>(H));
    CHECK(d.max < 5e-3 && d.mean < 1e-4 && d.over < static_cast<size_t>(H) / 100, "outside the golden tolerance");
}

// golden_test.go:122-201: SiLU of the golden 11008 inputs: max |d| < 5e-3,
// mean < 1e-4, fewer than 1% of elements off by more than 1e-3.
void TestSiLUGolden() {
    const std::vector<float> x = LoadGolden("silu_input.bin"), want = LoadGolden("silu_output.bin");
    CHECK(x.size() == want.size(), "golden sizes %zu %zu", x.size(), want.size());
    const int64_t n = static_cast<int64_t>(x.size());
    Owned in({n}, ng::Dtype::FP16), out({n}, ng::Dtype::FP16);
    NoError(ng::CopyToDevice(in.get(), x), "CopyToDevice");
    NoError(ng::SiLU(out.get(), in.get()), "SiLU");
    std::vector<float> got(n);
    NoError(ng::CopyToHost(got, out.get()), "CopyToHost");
    const DiffStats d = Diff(got, want, 1e-3);
    std::printf("  max_diff %.3e, avg_diff %.3e, errors %zu/%lld\n", d.max, d.mean, d.over, static_cast<long long>(n));
    CHECK(d.max < 5e-3 && d.mean < 1e-4 && d.over < static_cast<size_t>(n) / 100, "outside the golden tolerance");
}

// The bf16 wrappers (gpu.go:1329-1354; the Go suites hold no test of them):
// gfx950 reports bf16 support, and values exact in both formats convert to
// the bf16 pattern (the top half of their fp32 bits) and back unchanged.
void TestBF16Conversion() {
    bool supported = false;
    NoError(ng::CheckBF16Support(&supported), "CheckBF16Support");
    CHECK(supported, "bf16 reported unsupported");
    std::vector<float> x;
    for (int i = -1024; i <= 1024; i += 8) x.push_back(static_cast<float>(i) / 64.0f);
    for (int e = -14; e <= 15; ++e) x.push_back(std::ldexp(1.0f, e));
    const int n = static_cast<int>(x.size());
    Owned h({n}, ng::Dtype::FP16), b({2 * n}, ng::Dtype::INT8), back({n}, ng::Dtype::FP16);
    NoError(ng::CopyToDevice(h.get(), x), "CopyToDevice");
    NoError(ng::FP16ToBF16(b->Data, h->Data, n), "FP16ToBF16");
    NoError(ng::BF16ToFP16(back->Data, b->Data, n), "BF16ToFP16");
    NoError(ng::SyncDevice(), "SyncDevice");
    std::vector<int8_t> bytes(2 * n);
    std::vector<float> res(n);
    NoError(ng::CopyToHostINT8(bytes, b.get()), "CopyToHostINT8");
    NoError(ng::CopyToHost(res, back.get()), "CopyToHost");
    for (int i = 0; i < n; ++i) {
        uint32_t f;
        std::memcpy(&f, &x[i], 4);
        uint16_t got;
        std::memcpy(&got, &bytes[2 * i], 2);
        CHECK(got == (f >> 16), "bf16(%g) = 0x%04x, want 0x%04x", x[i], got, f >> 16);
        CHECK(res[i] == x[i], "fp16(bf16(%g)) = %g", x[i], res[i]);
    }
}

// cgo_test.go:141-159 and the wrappers' argument checks: each failure comes
// back as the Go wrapper's error text, and FreeTensor of an unallocated
// tensor is a no-op.
void TestCGOErrorHandling() {
    ng::Tensor bad = ng::NewTensor({1}, ng::Dtype::FP16, 999);
    WantError(ng::AllocateTensor(&bad), "invalid device ID: 999", "AllocateTensor(device 999)");
    ng::Tensor nil;
    ng::FreeTensor(&nil);
    ng::FreeTensor(nullptr);
    WantError(ng::CopyToDevice(&nil, {1.0f}), "tensor not allocated", "CopyToDevice(unallocated)");
    WantError(ng::AllocateTensor(nullptr), "tensor is nil", "AllocateTensor(nil)");
    ng::Tensor zero = ng::NewTensor({0}, ng::Dtype::FP16);
    WantError(ng::AllocateTensor(&zero), "tensor dimension 0 must be positive, got 0", "AllocateTensor([0])");
    ng::Tensor empty = ng::NewTensor({}, ng::Dtype::FP16);
    WantError(ng::AllocateTensor(&empty), "tensor shape cannot be empty", "AllocateTensor([])");

    Owned t({4}, ng::Dtype::FP16);
    WantError(ng::CopyToDevice(t.get(), {1.0f, 2.0f}), "data size 2 < tensor size 4", "CopyToDevice(short)");
    std::vector<float> shorter(3);
    WantError(ng::CopyToHost(shorter, t.get()), "buffer size 3 < tensor size 4", "CopyToHost(short)");
    WantError(ng::CopyToDeviceINT8(t.get(), std::vector<int8_t>(8)), "tensor dtype must be INT8",
              "CopyToDeviceINT8(fp16 tensor)");
    WantError(ng::RoPE(t.get(), t.get(), {0}, 128), "input must have 4 dimensions", "RoPE(1-d)");
    WantError(ng::RMSNorm(nullptr, t.get(), t.get(), 1e-6f), "nil tensor", "RMSNorm(nil)");
    ng::Tensor unalloc = ng::NewTensor({4}, ng::Dtype::FP16);
    WantError(ng::RMSNorm(t.get(), &unalloc, t.get(), 1e-6f), "tensor not allocated", "RMSNorm(unallocated)");
    WantError(ng::SiLU(t.get(), nullptr), "nil tensor", "SiLU(nil)");
    WantError(ng::GEMMINT8(t.get(), t.get(), nullptr, t.get(), true), "nil tensor", "GEMMINT8(nil)");
    // An error the library reports is formatted with its code: the kernel
    // rejects a null pointer with -1.
    WantError(ng::SiLU(&unalloc, t.get()), "SiLU failed: -1", "SiLU(null output)");
    // Shapes the wrappers' shape rules cannot read (Go would index out of
    // range and panic) come back as errors.
    ng::Tensor flat = t.t, scalarless = t.t;
    scalarless.Shape.clear();
    WantError(ng::RMSNorm(t.get(), &scalarless, t.get(), 1e-6f), "RMSNorm: tensor has 0 dimensions",
              "RMSNorm(no dimensions)");
    WantError(ng::GEMMINT8(t.get(), &flat, t.get(), t.get(), true), "GEMM INT8: tensor has 1 dimensions",
              "GEMMINT8(1-d A)");
    WantError(ng::GEMMFP16(t.get(), t.get(), &flat, false, false), "GEMM FP16: tensor has 1 dimensions",
              "GEMMFP16(1-d B)");
    WantError(ng::QuantizeWeights(t.get(), t.get(), &flat), "quantize weights: tensor has 1 dimensions",
              "QuantizeWeights(1-d)");
    // Tensors smaller than the call touches are refused before any launch.
    Owned q4({1, 2, 4, 64}, ng::Dtype::FP16), big({1024}, ng::Dtype::FP16);
    WantError(ng::RoPE(q4.get(), q4.get(), {0}, 64), "RoPE: positions has 1 elements, the call needs 2",
              "RoPE(short positions)");
    WantError(ng::RoPE(q4.get(), q4.get(), {0, 1}, 128), "RoPE: input has 512 elements, the call needs 1024",
              "RoPE(head_dim past the tensor)");
    WantError(ng::SiLU(t.get(), big.get()), "SiLU: output has 4 elements, the call needs 1024", "SiLU(short output)");
    WantError(ng::Add(big.get(), big.get(), t.get()), "Add: b has 4 elements, the call needs 1024", "Add(short b)");
    Owned a8({2, 64}, ng::Dtype::FP16), b8({16, 32}, ng::Dtype::INT8), c8({2, 16}, ng::Dtype::FP16),
        s8({16}, ng::Dtype::FP32);
    WantError(ng::GEMMINT8(c8.get(), a8.get(), b8.get(), s8.get(), true),
              "GEMM INT8: b has 512 elements, the call needs 1024", "GEMMINT8(K of B short)");
    WantError(ng::RMSNorm(big.get(), big.get(), t.get(), 1e-6f), "RMSNorm: weight has 4 elements, the call needs 1024",
              "RMSNorm(short weight)");
}

void GemmFP16Case(bool transposeA) {
    const int M = 32, K = 128, N = 64;
    std::mt19937 rng(42);
    const std::vector<float> da = Uniform(rng, static_cast<size_t>(M) * K);
    const std::vector<float> db = Uniform(rng, static_cast<size_t>(K) * N);
    Owned a(transposeA ? std::vector<int64_t>{K, M} : std::vector<int64_t>{M, K}, ng::Dtype::FP16);
    Owned b({K, N}, ng::Dtype::FP16), c({M, N}, ng::Dtype::FP16);
    NoError(ng::CopyToDevice(a.get(), da), "CopyToDevice");
    NoError(ng::CopyToDevice(b.get(), db), "CopyToDevice");
    NoError(ng::GEMMFP16(c.get(), a.get(), b.get(), transposeA, false), "GEMMFP16");
    std::vector<float> res(static_cast<size_t>(M) * N);
    NoError(ng::CopyToHost(res, c.get()), "CopyToHost");
    std::vector<float> am = da;
    if (transposeA)
        for (int k = 0; k < K; ++k)
            for (int m = 0; m < M; ++m) am[static_cast<size_t>(m) * K + k] = da[static_cast<size_t>(k) * M + m];
    const std::vector<float> ref = CpuMatmul(am, db, M, K, N);
    double dmax = 0;
    for (size_t i = 0; i < res.size(); ++i) dmax = std::max(dmax, std::fabs(static_cast<double>(res[i]) - ref[i]));
    std::printf("  maxDiff %g\n", dmax);
    CHECK(dmax < 0.1, "GEMM FP16 max diff %g exceeds 0.1", dmax);
}

// matmul_test.go:20-94: [32, 128] @ [128, 64], U(-1, 1), max |d| < 0.1.
void TestGEMMFP16() { GemmFP16Case(false); }

// matmul_test.go:182-260: A stored [K, M] and read transposed.
void TestGEMMTranspose() { GemmFP16Case(true); }

// matmul_test.go:96-179 in both weight layouts: A [32, 128] U(-1, 1), codes
// U{-128..127}, scales 0.01, max |d| < 5e-2 against the fp32 CPU product.
void TestGEMMINT8() {
    const int M = 32, K = 128, N = 64;
    std::mt19937 rng(42);
    const std::vector<float> da = Uniform(rng, static_cast<size_t>(M) * K);
    std::uniform_int_distribution<int> u(-128, 127);
    for (bool transposeB : {false, true}) {
        std::vector<int8_t> codes(static_cast<size_t>(K) * N);
        for (auto& c : codes) c = static_cast<int8_t>(u(rng));
        const std::vector<float> scale(N, 0.01f);
        Owned a({M, K}, ng::Dtype::FP16), c({M, N}, ng::Dtype::FP16), sc({N}, ng::Dtype::FP32);
        Owned b(transposeB ? std::vector<int64_t>{N, K} : std::vector<int64_t>{K, N}, ng::Dtype::INT8);
        NoError(ng::CopyToDevice(a.get(), da), "CopyToDevice");
        NoError(ng::CopyToDeviceINT8(b.get(), codes), "CopyToDeviceINT8");
        NoError(ng::CopyToDevice(sc.get(), scale), "CopyToDevice");
        NoError(ng::GEMMINT8(c.get(), a.get(), b.get(), sc.get(), transposeB), "GEMMINT8");
        std::vector<float> res(static_cast<size_t>(M) * N);
        NoError(ng::CopyToHost(res, c.get()), "CopyToHost");
        std::vector<float> w(static_cast<size_t>(K) * N);  // [K, N]
        for (int k = 0; k < K; ++k)
            for (int n = 0; n < N; ++n)
                w[static_cast<size_t>(k) * N + n] =
                    codes[transposeB ? static_cast<size_t>(n) * K + k : static_cast<size_t>(k) * N + n] * scale[n];
        const std::vector<float> ref = CpuMatmul(da, w, M, K, N);
        double dmax = 0;
        for (size_t i = 0; i < res.size(); ++i)
            dmax = std::max(dmax, std::fabs(static_cast<double>(res[i]) - ref[i]));
        std::printf("  transposeB=%d maxDiff %g\n", transposeB, dmax);
        CHECK(dmax < 5e-2, "GEMM INT8 (transposeB=%d) max diff %g", transposeB, dmax);
    }
}

// cgo_test.go:244-271: SyncDevice on an idle device costs under 10 us per call.
void TestCGOOverheadValidation() {
    for (int i = 0; i < 100; ++i) NoError(ng::SyncDevice(), "SyncDevice");
    const int n = 10000;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n; ++i) (void)ng::SyncDevice();
    const double us =
        std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / n;
    std::printf("  SyncDevice: %.3f us per call\n", us);
    CHECK(us < 10.0, "SyncDevice takes %.2f us per call", us);
}

// Runs fn(i) on `threads` threads; the first failure message is rethrown.
void RunThreads(int threads, const std::function<void(int)>& fn) {
    std::vector<std::string> errors(threads);
    std::vector<std::thread> pool;
    for (int i = 0; i < threads; ++i)
        pool.emplace_back([&, i] {
            try {
                fn(i);
            } catch (const std::exception& e) {
                errors[i] = e.what();
            }
        });
    for (auto& t : pool) t.join();
    for (int i = 0; i < threads; ++i)
        if (!errors[i].empty()) throw Failure("thread " + std::to_string(i) + ": " + errors[i]);
}

// cgo_test.go:274-313: 10 threads x 100 rounds of allocate / copy in / copy
// out / free of a [256] fp16 tensor; every round trip is the fp16 rounding.
void TestCGOConcurrentCalls() {
    RunThreads(10, [](int seed) {
        std::mt19937 rng(seed);
        std::normal_distribution<float> g;
        std::vector<float> data(256), want(256);
        for (int i = 0; i < 256; ++i) {
            data[i] = g(rng);
            want[i] = static_cast<float>(RoundToHalf(data[i]));
        }
        for (int r = 0; r < 100; ++r) {
            Owned t({256}, ng::Dtype::FP16);
            NoError(ng::CopyToDevice(t.get(), data), "CopyToDevice");
            std::vector<float> back(256);
            NoError(ng::CopyToHost(back, t.get()), "CopyToHost");
            CHECK(back == want, "round %d: round trip differs", r);
        }
    });
}

// Six threads call GEMMINT8 at once on the library's one launch stream,
// through the split-K path (M = 40: two kernels per call sharing the stream's
// partial-sum buffer) and the library path (M = 200: the stream's fp16 weight
// copy). Operands are exact in fp16 and the products in fp32, so every
// output is the fp16 rounding of the exact product.
void TestConcurrentGEMMINT8() {
    const int K = 512, N = 256;
    RunThreads(6, [&](int seed) {
        std::mt19937 rng(100 + seed);
        std::uniform_int_distribution<int> ua(-64, 64), uc(-128, 127);
        for (int M : {40, 200, 40, 200}) {
            std::vector<float> da(static_cast<size_t>(M) * K);
            for (auto& v : da) v = static_cast<float>(ua(rng)) / 64.0f;
            std::vector<int8_t> codes(static_cast<size_t>(N) * K);
            for (auto& c : codes) c = static_cast<int8_t>(uc(rng));
            const float s = 1.0f / 128.0f;
            Owned a({M, K}, ng::Dtype::FP16), c({M, N}, ng::Dtype::FP16);
            Owned b({N, K}, ng::Dtype::INT8), sc({N}, ng::Dtype::FP32);
            NoError(ng::CopyToDevice(a.get(), da), "CopyToDevice");
            NoError(ng::CopyToDeviceINT8(b.get(), codes), "CopyToDeviceINT8");
            NoError(ng::CopyToDevice(sc.get(), std::vector<float>(N, s)), "CopyToDevice");
            for (int r = 0; r < 5; ++r) NoError(ng::GEMMINT8(c.get(), a.get(), b.get(), sc.get(), true), "GEMMINT8");
            std::vector<float> res(static_cast<size_t>(M) * N);
            NoError(ng::CopyToHost(res, c.get()), "CopyToHost");
            for (int m = 0; m < M; ++m)
                for (int n = 0; n < N; ++n) {
                    double acc = 0;
                    for (int k = 0; k < K; ++k)
                        acc += static_cast<double>(da[static_cast<size_t>(m) * K + k]) *
                               codes[static_cast<size_t>(n) * K + k] * s;
                    const float want = static_cast<float>(RoundToHalf(acc));
                    CHECK(res[static_cast<size_t>(m) * N + n] == want, "M=%d [%d,%d]: %g, want %g", M, m, n,
                          res[static_cast<size_t>(m) * N + n], want);
                }
        }
    });
}

// cgo_test.go:16-34: shutdown resets the device; init works again after it,
// and a kernel runs on the re-initialised device.
void TestCGOInitShutdown() {
    ng::ShutdownGPU();
    NoError(ng::InitGPU(0), "InitGPU after ShutdownGPU");
    ng::DeviceInfo info;
    NoError(ng::GetDeviceInfo(&info), "GetDeviceInfo");
    TestAddKernel();
    TestGEMMINT8();
    ng::ShutdownGPU();
    NoError(ng::InitGPU(0), "InitGPU after the second ShutdownGPU");
}

struct Case {
    const char* name;
    void (*fn)();
};

// TestCGOInitShutdown resets the device and comes last.
const Case kCases[] = {
    {"TestDeviceInfo", TestDeviceInfo},
    {"TestRMSNorm", TestRMSNorm},
    {"TestSiLU", TestSiLU},
    {"TestRMSNormGolden", TestRMSNormGolden},
    {"TestSiLUGolden", TestSiLUGolden},
    {"TestRoPE", TestRoPE},
    {"TestAddKernel", TestAddKernel},
    {"TestQuantizePerTensor", TestQuantizePerTensor},
    {"TestDequantizePerTensor", TestDequantizePerTensor},
    {"TestQuantizeWeights", TestQuantizeWeights},
    {"TestCopyFP16RoundToNearestEven", TestCopyFP16RoundToNearestEven},
    {"TestEmbeddingLookup", TestEmbeddingLookup},
    {"TestBF16Conversion", TestBF16Conversion},
    {"TestCGOErrorHandling", TestCGOErrorHandling},
    {"TestGEMMFP16", TestGEMMFP16},
    {"TestGEMMTranspose", TestGEMMTranspose},
    {"TestGEMMINT8", TestGEMMINT8},
    {"TestCGOOverheadValidation", TestCGOOverheadValidation},
    {"TestCGOConcurrentCalls", TestCGOConcurrentCalls},
    {"TestConcurrentGEMMINT8", TestConcurrentGEMMINT8},
    {"TestCGOInitShutdown", TestCGOInitShutdown},
};

}  // namespace

int main(int argc, char** argv) {
    std::vector<std::string> want;
    {
        // Default golden directory: tests/golden/reference_kernels beside this
        // program's neurogrid_amd/lib/.
        char exe[4096];
        const ssize_t len = readlink("/proc/self/exe", exe, sizeof(exe) - 1);
        std::string dir = len > 0 ? std::string(exe, static_cast<size_t>(len)) : std::string(argv[0]);
        dir = dir.substr(0, dir.find_last_of('/') == std::string::npos ? 0 : dir.find_last_of('/'));
        g_golden_dir = dir + "/../../tests/golden/reference_kernels";
    }
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--list") == 0) {
            for (const Case& c : kCases) std::printf("%s\n", c.name);
            return 0;
        }
        if (std::strcmp(argv[i], "--golden") == 0 && i + 1 < argc) {
            g_golden_dir = argv[++i];
            continue;
        }
        want.emplace_back(argv[i]);
    }
    for (const std::string& w : want) {
        bool known = false;
        for (const Case& c : kCases) known |= w == c.name;
        if (!known) {
            std::fprintf(stderr, "unknown test %s\n", w.c_str());
            return 2;
        }
    }
    if (ng::Error e = ng::InitGPU(0)) {
        std::printf("FAIL InitGPU: %s\n", e.message().c_str());
        return 1;
    }
    int failed = 0, ran = 0;
    for (const Case& c : kCases) {
        if (!want.empty() && std::find(want.begin(), want.end(), c.name) == want.end()) continue;
        std::printf("RUN  %s\n", c.name);
        std::fflush(stdout);
        const auto t0 = std::chrono::steady_clock::now();
        try {
            c.fn();
            NoError(ng::SyncDevice(), "SyncDevice after the test");
            const double ms =
                std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            std::printf("PASS %s (%.1f ms)\n", c.name, ms);
        } catch (const std::exception& e) {
            std::printf("FAIL %s: %s\n", c.name, e.what());
            ++failed;
        }
        ++ran;
        std::fflush(stdout);
    }
    ng::ShutdownGPU();
    std::printf("%d of %d tests passed\n", ran - failed, ran);
    return failed;
}
