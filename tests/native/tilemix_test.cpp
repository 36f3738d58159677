// Native test driver for the HIP TileMix library, exercising the reference's
// C++ API (include/attention_fused.h) the way the reference test binary does
// (src/tests/tilemix_test.cu). Modes, as in tilemix_test.cu:617-631:
//   tilemix_test                 CPU checks + GPU checks
//   tilemix_test --cpu-only      CPU checks only (no HIP runtime call)
//   tilemix_test --export-json F also writes the dense cases as JSONL fixtures
// The checker is the C oracle (oracle/tilemix_oracle.h), linked as test code.

#include "attention_fused.h"
#include "tilemix_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

void hip_ok(hipError_t status) {
    if (status != hipSuccess) throw std::runtime_error(hipGetErrorString(status));
}

void expect(bool condition, const char* message) {
    if (!condition) throw std::runtime_error(message);
}

template <class T>
struct Buffer {
    T* ptr = nullptr;
    std::size_t count = 0;
    explicit Buffer(std::size_t n) : count(n) { hip_ok(hipMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T))); }
    ~Buffer() { (void)hipFree(ptr); }
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    void put(const T* host, hipStream_t s) { hip_ok(hipMemcpyAsync(ptr, host, count * sizeof(T), hipMemcpyHostToDevice, s)); }
    std::vector<T> get() const {
        std::vector<T> host(count);
        hip_ok(hipMemcpy(host.data(), ptr, count * sizeof(T), hipMemcpyDeviceToHost));
        return host;
    }
};

struct StreamHandle {
    hipStream_t value = nullptr;
    explicit StreamHandle(bool use_default) {
        if (!use_default) hip_ok(hipStreamCreateWithFlags(&value, hipStreamNonBlocking));
    }
    ~StreamHandle() { if (value) (void)hipStreamDestroy(value); }
};

struct Inputs {
    std::vector<std::uint16_t> q, k, v;
};

Inputs make_inputs(int m, int n, int d, const char* pattern) {
    Inputs in{std::vector<std::uint16_t>(static_cast<std::size_t>(m) * d),
              std::vector<std::uint16_t>(static_cast<std::size_t>(n) * d),
              std::vector<std::uint16_t>(static_cast<std::size_t>(n) * d)};
    expect(tmo_make_inputs(m, n, d, pattern, in.q.data(), in.k.data(), in.v.data()) == 0, "unknown input pattern");
    return in;
}

const __half* as_half(const std::vector<std::uint16_t>& bits) { return reinterpret_cast<const __half*>(bits.data()); }

// |a - e| <= atol + rtol |e| (the reference's comparison rule).
template <class T>
void compare(const std::vector<T>& actual, const std::vector<double>& expected, const char* label,
             double atol, double rtol) {
    expect(!actual.empty() && actual.size() == expected.size(), "output shape mismatch");
    double max_abs = 0.0, max_rel = 0.0, squares = 0.0;
    for (std::size_t i = 0; i < actual.size(); ++i) {
        const double a = static_cast<double>(actual[i]);
        const double error = std::fabs(a - expected[i]);
        if (!std::isfinite(a) || !std::isfinite(expected[i]) || error > atol + rtol * std::fabs(expected[i])) {
            std::fprintf(stderr, "%s mismatch at %zu: got %.17g expected %.17g\n", label, i, a, expected[i]);
            throw std::runtime_error("TileMix comparison failed");
        }
        max_abs = std::max(max_abs, error);
        max_rel = std::max(max_rel, error / std::max(std::fabs(expected[i]), atol));
        squares += error * error;
    }
    std::printf("PASS %s atol=%.1g rtol=%.1g max_abs_error=%.9g max_rel_error=%.9g rms_error=%.9g\n", label, atol,
                rtol, max_abs, max_rel, std::sqrt(squares / actual.size()));
}

// ------------------------------------------------------------------ CPU
void cpu_checks() {
    const __half x = __float2half(1.0f);
    float out = 0.0f;
    expect(launch_fused_fp16_attention(nullptr, &x, &x, &out, 1, 1, 1, 1.0f) == hipErrorInvalidValue, "null Q accepted");
    expect(launch_fused_fp16_attention(&x, nullptr, &x, &out, 1, 1, 1, 1.0f) == hipErrorInvalidValue, "null K accepted");
    expect(launch_fused_fp16_attention(&x, &x, nullptr, &out, 1, 1, 1, 1.0f) == hipErrorInvalidValue, "null V accepted");
    expect(launch_fused_fp16_attention(&x, &x, &x, nullptr, 1, 1, 1, 1.0f) == hipErrorInvalidValue, "null O accepted");
    for (int bad : {0, -1}) {
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, bad, 1, 1, 1.0f) == hipErrorInvalidValue, "bad M accepted");
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, bad, 1, 1.0f) == hipErrorInvalidValue, "bad N accepted");
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, bad, 1.0f) == hipErrorInvalidValue, "bad d accepted");
    }
    for (int d : {129, std::numeric_limits<int>::max()})
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, d, 1.0f) == hipErrorNotSupported, "d > 128 accepted");
    for (float scale : {std::numeric_limits<float>::quiet_NaN(), std::numeric_limits<float>::infinity(),
                        -std::numeric_limits<float>::infinity()})
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, 1, scale) == hipErrorInvalidValue,
               "non-finite scale accepted");
    static_assert(fused_fp16_shared_bytes(1) == 4608 && fused_fp16_shared_bytes(17) == 7168 &&
                  fused_fp16_shared_bytes(128) == 22528 && fused_fp16_shared_bytes(129) == 0);
    static_assert(kTileMixQQuantRows == 128 && kTileMixKQuantRows == 64 && tilemix_shared_bytes(128, true) == 28672 &&
                  tilemix_shared_bytes(17, true) == 8704);
    expect(tilemix_shared_bytes_c(128, 1) == 28672 && tilemix_shared_bytes_c(17, 1) == 8704, "C-ABI sizing mirror");
    std::int8_t byte = 0;
    __half scale_out;
    expect(quantize_tilemix_qk(nullptr, &x, &byte, &byte, &scale_out, &scale_out, 1, 1, 1) == hipErrorInvalidValue,
           "null quantizer input accepted");
    expect(quantize_tilemix_qk(&x, &x, nullptr, &byte, &scale_out, &scale_out, 1, 1, 1) == hipErrorInvalidValue,
           "null quantizer output accepted");
    expect(quantize_tilemix_qk(&x, &x, &byte, &byte, nullptr, &scale_out, 1, 1, 1) == hipErrorInvalidValue,
           "null scale output accepted");
    expect(quantize_tilemix_qk(&x, &x, &byte, &byte, &scale_out, &scale_out, 0, 1, 1) == hipErrorInvalidValue,
           "empty quantizer input accepted");
    expect(quantize_tilemix_qk(&x, &x, &byte, &byte, &scale_out, &scale_out, 1, 1, 129) == hipErrorNotSupported,
           "quantizer d > 128 accepted");
    const TileMixQuantized partial{&byte};
    expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, 1, 1.0f, nullptr, {}, partial) == hipErrorInvalidValue,
           "partial quantized operands accepted");
    static_assert(tilemix_routing_word_count(17, 2048, 1) == 2 && tilemix_routing_word_count(17, 2049, 1) == 4 &&
                  tilemix_routing_word_count(17, 4097, 2) == 4 && tilemix_routing_word_count(17, 4097, 1) == 6 &&
                  tilemix_routing_word_count(17, std::numeric_limits<int>::max(), std::numeric_limits<int>::max()) == 2 &&
                  tilemix_routing_word_count(0, 1, 1) == 0 && tilemix_routing_word_count(1, 0, 1) == 0 &&
                  tilemix_routing_word_count(1, 1, 0) == 0);
    expect(tilemix_routing_word_count_c(17, 4097, 1) == 6 && tilemix_routing_word_count_c(1, 1, 0) == 0,
           "C-ABI routing mirror");
    for (int group : {0, -1}) {
        const TileMixRouting routing{nullptr, 0, group};
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, 1, 1.0f, nullptr, routing) == hipErrorInvalidValue,
               "non-positive group accepted");
    }
    const std::uint64_t word = 0;
    expect(launch_fused_fp16_attention(&x, &x, &x, &out, 1, 1, 1, 1.0f, nullptr, TileMixRouting{&word, 1, 1}) ==
               hipErrorInvalidValue, "routing without quantized operands accepted");
    for (const TileMixRouting routing : {TileMixRouting{nullptr, 1, 1}, TileMixRouting{&word, 0, 1},
                                        TileMixRouting{&word, 3, 1}})
        expect(launch_fused_fp16_attention(&x, &x, &x, &out, 17, 2049, 1, 1.0f, nullptr, routing) == hipErrorInvalidValue,
               "null or undersized routing mask accepted");
    std::puts("PASS TileMix API validation and sizing helpers (no HIP runtime call)");

    // Closed forms of the score patterns (tilemix_test.cu:237-260) against the fp64 oracle.
    for (const char* pattern : {"rising", "falling", "alternating", "late-extreme", "negative"}) {
        const int n = std::string(pattern) == "alternating" ? 129 : 65;
        const Inputs in = make_inputs(17, n, 1, pattern);
        std::vector<double> actual(17);
        expect(tmo_attention(in.q.data(), in.k.data(), in.v.data(), 17, n, 1, actual.data()) == 0, "oracle failed");
        double expected = 0.0;
        const std::string p = pattern;
        if (p == "rising") {
            const double a = 32 * std::exp(-8.0), b = 32 * std::exp(-4.0);
            expected = (a - b + 2) / (a + b + 1);
        } else if (p == "falling") {
            const double b = 32 * std::exp(-4.0), c = std::exp(-8.0);
            expected = (32 - b + 2 * c) / (32 + b + c);
        } else if (p == "alternating") {
            const double a = 32 * std::exp(-10.0), b = 32 * std::exp(-6.0), c = 32 * std::exp(-12.0), e = 32 * std::exp(-2.0);
            expected = (a - b + 2 * c - 2 * e + 3) / (a + b + c + e + 1);
        } else if (p == "late-extreme") {
            expected = 3.0;
        } else {
            for (std::uint16_t value : in.v) expected += tmo_half_to_float(value);
            expected /= n;
        }
        compare(actual, std::vector<double>(17, expected), pattern, 1e-12, 1e-12);
    }
}

// ------------------------------------------------------------------ GPU
struct Shape {
    int m, n, d;
    const char* pattern;
    bool default_stream;
};

void dense_case(const Shape& s, std::ostream* fixtures) {
    const std::size_t count = static_cast<std::size_t>(s.m) * s.d, kv = static_cast<std::size_t>(s.n) * s.d;
    const Inputs in = make_inputs(s.m, s.n, s.d, s.pattern);
    std::vector<double> expected(count);
    expect(tmo_attention(in.q.data(), in.k.data(), in.v.data(), s.m, s.n, s.d, expected.data()) == 0, "oracle failed");
    constexpr float guard = -12345.25f;
    std::vector<float> host(count + 2, std::numeric_limits<float>::quiet_NaN());
    host.front() = host.back() = guard;
    Buffer<std::uint16_t> q(count), k(kv), v(kv);
    Buffer<float> out(count + 2);
    StreamHandle stream(s.default_stream);
    q.put(in.q.data(), stream.value);
    k.put(in.k.data(), stream.value);
    v.put(in.v.data(), stream.value);
    out.put(host.data(), stream.value);
    hip_ok(launch_fused_fp16_attention(reinterpret_cast<const __half*>(q.ptr), reinterpret_cast<const __half*>(k.ptr),
                                       reinterpret_cast<const __half*>(v.ptr), out.ptr + 1, s.m, s.n, s.d,
                                       1.0f / std::sqrt(static_cast<float>(s.d)), stream.value));
    hip_ok(hipStreamSynchronize(stream.value));
    host = out.get();
    expect(host.front() == guard && host.back() == guard, "output guard overwritten");
    std::printf("Case M=%d N=%d d=%d pattern=%s stream=%s\n", s.m, s.n, s.d, s.pattern,
                s.default_stream ? "default" : "nonblocking");
    compare(std::vector<float>(host.begin() + 1, host.end() - 1), expected, "TileMix vs CPU FP64", 1e-5, 1e-4);
    expect(q.get() == in.q && k.get() == in.k && v.get() == in.v, "kernel modified a Q/K/V input");
    if (fixtures) {
        auto& f = *fixtures;
        f << std::setprecision(std::numeric_limits<float>::max_digits10) << "{\"m\":" << s.m << ",\"n\":" << s.n
          << ",\"d\":" << s.d << ",\"pattern\":\"" << s.pattern << "\"";
        const auto halves = [&](const char* name, const std::vector<std::uint16_t>& values) {
            f << ",\"" << name << "\":[";
            for (std::size_t i = 0; i < values.size(); ++i) f << (i ? "," : "") << tmo_half_to_float(values[i]);
            f << "]";
        };
        halves("q", in.q);
        halves("k", in.k);
        halves("v", in.v);
        f << ",\"o\":[";
        for (std::size_t i = 1; i <= count; ++i) f << (i > 1 ? "," : "") << host[i];
        f << "]}\n";
        expect(static_cast<bool>(f), "failed to write a JSON fixture");
    }
}

void routing_case(const Shape& s, int group, const std::string& pattern) {
    const std::size_t qtiles = (s.m + 15) / 16, ktiles = (s.n + 31) / 32;
    const std::size_t groups = (ktiles + group - 1) / group, wpr = (groups + 63) / 64;
    std::vector<std::uint64_t> words(qtiles * wpr, ~std::uint64_t{0});
    std::vector<std::uint8_t> bits(qtiles * ktiles);
    for (std::size_t row = 0; row < qtiles; ++row) {
        std::size_t tile = 0;
        for (std::size_t grp = 0; grp < groups; ++grp) {
            const bool bit = pattern == "int8-requested" || (pattern == "mixed" && (grp + row + grp / 64) % 2 == 0);
            const std::uint64_t flag = std::uint64_t{1} << (grp % 64);
            std::uint64_t& w = words[row * wpr + grp / 64];
            w = bit ? (w | flag) : (w & ~flag);
            for (int r = 0; r < group && tile < ktiles; ++r, ++tile) bits[row * ktiles + tile] = bit;
        }
    }
    expect(words.size() == tilemix_routing_word_count(s.m, s.n, group), "routing layout mismatch");
    const Inputs in = make_inputs(s.m, s.n, s.d, s.pattern);
    const std::size_t count = in.q.size(), kv = in.k.size();
    std::vector<std::int8_t> q8_ref(count), k8_ref(kv);
    std::vector<std::uint16_t> qs_ref((s.m + 127) / 128), ks_ref((s.n + 63) / 64);
    tmo_quantize(in.q.data(), s.m, s.d, 128, q8_ref.data(), qs_ref.data());
    tmo_quantize(in.k.data(), s.n, s.d, 64, k8_ref.data(), ks_ref.data());
    StreamHandle stream(false);
    Buffer<std::uint16_t> q(count), k(kv), v(kv), qs(qs_ref.size()), ks(ks_ref.size());
    Buffer<std::int8_t> q8(count), k8(kv);
    Buffer<float> out(count);
    Buffer<std::uint64_t> mask(words.size());
    Buffer<std::uint8_t> trace(bits.size());
    Buffer<std::int32_t> dots(static_cast<std::size_t>(s.m) * s.n);
    q.put(in.q.data(), stream.value);
    k.put(in.k.data(), stream.value);
    v.put(in.v.data(), stream.value);
    mask.put(words.data(), stream.value);
    constexpr std::int32_t dot_guard = 0x2468ace;
    const std::vector<std::int32_t> dot_fill(dots.count, dot_guard);
    dots.put(dot_fill.data(), stream.value);
    const auto hq = reinterpret_cast<const __half*>(q.ptr);
    const auto hk = reinterpret_cast<const __half*>(k.ptr);
    const auto hv = reinterpret_cast<const __half*>(v.ptr);
    hip_ok(quantize_tilemix_qk(hq, hk, q8.ptr, k8.ptr, reinterpret_cast<__half*>(qs.ptr), reinterpret_cast<__half*>(ks.ptr),
                               s.m, s.n, s.d, stream.value));
    const float scale = 1.0f / std::sqrt(static_cast<float>(s.d));
    hip_ok(launch_fused_fp16_attention(hq, hk, hv, out.ptr, s.m, s.n, s.d, scale, stream.value));
    hip_ok(hipStreamSynchronize(stream.value));
    const std::vector<float> baseline = out.get();
    const TileMixRouting routing{mask.ptr, words.size(), group, trace.ptr};
    const TileMixQuantized quantized{q8.ptr, k8.ptr, reinterpret_cast<const __half*>(qs.ptr),
                                     reinterpret_cast<const __half*>(ks.ptr), dots.ptr};
    hip_ok(launch_fused_fp16_attention(hq, hk, hv, out.ptr, s.m, s.n, s.d, scale, stream.value, routing, quantized));
    hip_ok(hipStreamSynchronize(stream.value));
    const std::vector<float> actual = out.get();
    if (std::none_of(bits.begin(), bits.end(), [](std::uint8_t b) { return b != 0; }))
        expect(std::memcmp(actual.data(), baseline.data(), actual.size() * sizeof(float)) == 0,
               "all-FP16 routing changed the un-routed output");
    const std::vector<std::int32_t> got_dots = dots.get();
    for (int query = 0; query < s.m; ++query)
        for (int key = 0; key < s.n; ++key) {
            const bool int8 = bits[(query / 16) * ktiles + key / 32] != 0;
            const std::int32_t want = int8 ? tmo_int8_dot(q8_ref.data(), k8_ref.data(), query, key, s.d) : dot_guard;
            expect(got_dots[static_cast<std::size_t>(query) * s.n + key] == want, "int32 dot mismatch");
        }
    expect(trace.get() == bits, "routing trace mismatch");
    expect(q8.get() == q8_ref && k8.get() == k8_ref && qs.get() == qs_ref && ks.get() == ks_ref,
           "quantized operands mismatch");
    std::vector<double> expected(count);
    tmo_tilemix(in.q.data(), in.k.data(), in.v.data(), q8_ref.data(), k8_ref.data(), qs_ref.data(), ks_ref.data(),
                bits.data(), s.m, s.n, s.d, scale, 0, nullptr, 0, expected.data());
    std::printf("Routing M=%d N=%d d=%d g=%d pattern=%s\n", s.m, s.n, s.d, group, pattern.c_str());
    compare(actual, expected, "mixed FP16/INT8 vs fp64 TileMix oracle", 1e-5, 1e-4);
}

void gpu_checks(std::ostream* fixtures) {
    int device = 0;
    hipDeviceProp_t properties{};
    hip_ok(hipGetDevice(&device));
    hip_ok(hipGetDeviceProperties(&properties, device));
    int driver = 0, runtime = 0;
    hip_ok(hipDriverGetVersion(&driver));
    hip_ok(hipRuntimeGetVersion(&runtime));
    std::printf("GPU=%s arch=%s driver=%d runtime=%d\n", properties.name, properties.gcnArchName, driver, runtime);
    int cases = 0;
    for (int d : {1, 15, 16, 17, 31, 32, 33, 49, 63, 64, 65, 81, 97, 113, 127, 128}) {
        dense_case({3, 33, d, "random", false}, fixtures);
        ++cases;
    }
    const Shape shapes[] = {{1, 1, 1, "random", false}, {3, 5, 7, "random", false}, {15, 31, 15, "random", false},
                            {16, 32, 16, "random", false}, {17, 33, 17, "random", false}, {31, 63, 31, "random", false},
                            {32, 64, 32, "random", false}, {33, 65, 33, "random", false}, {35, 67, 65, "random", false},
                            {17, 65, 128, "random", false}, {17, 1, 128, "random", false}, {17, 33, 17, "random", true},
                            {17, 65, 1, "rising", false}, {17, 65, 1, "falling", false}, {17, 129, 1, "alternating", false},
                            {17, 65, 1, "late-extreme", false}, {17, 33, 1, "negative", false}, {17, 33, 17, "zeros", false},
                            {17, 33, 17, "uniform", false}, {17, 33, 17, "zero-v", false}, {17, 65, 17, "constant-v", false},
                            {2, 32, 17, "cancellation", false}, {17, 33, 1, "large-dot", false},
                            {3, 2051, 17, "random", false}, {1, 4097, 128, "uniform", false}};
    for (const Shape& s : shapes) {
        dense_case(s, fixtures);
        ++cases;
    }
    int routed = 0;
    const std::pair<Shape, int> routing_shapes[] = {
        {{35, 67, 17, "random", false}, 2}, {{17, 2049, 5, "random", false}, 1}, {{17, 4099, 5, "random", false}, 2},
        {{35, 163, 17, "random", false}, 3}, {{17, 65, 17, "random", false}, std::numeric_limits<int>::max()},
        {{129, 131, 17, "block-outliers", false}, 1}, {{17, 33, 128, "max-int8", false}, 1},
        {{3, 33, 64, "random", false}, 1}, {{3, 33, 128, "random", false}, 1}};
    for (const auto& [shape, group] : routing_shapes)
        for (const char* pattern : {"fp16", "int8-requested", "mixed"}) {
            routing_case(shape, group, pattern);
            ++routed;
        }
    std::printf("PASS TileMix native suite: %d FP64-reference cases + %d routing cases\n", cases, routed);
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const bool cpu_only = argc == 2 && std::string(argv[1]) == "--cpu-only";
        const bool export_json = argc == 3 && std::string(argv[1]) == "--export-json";
        if (argc != 1 && !cpu_only && !export_json)
            throw std::invalid_argument("usage: tilemix_test [--cpu-only | --export-json FILE]");
        std::ofstream fixtures;
        if (export_json) {
            fixtures.open(argv[2]);
            expect(static_cast<bool>(fixtures), "could not open the JSON fixture file");
        }
        std::puts("TileMix native tests (HIP, gfx950): FP16/INT8 score routes, 128/64-row Q/K quantization.");
        cpu_checks();
        if (!cpu_only) gpu_checks(export_json ? &fixtures : nullptr);
        return 0;
    } catch (const std::exception& error) {
        std::fprintf(stderr, "ERROR: %s\n", error.what());
        return 1;
    }
}
