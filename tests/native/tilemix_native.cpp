// Native check program for the HIP TileMix library, driven through the
// reference's own C++ entry points (include/attention_fused.h) so that it
// exercises the drop-in boundary exactly as a reference caller would. The
// checker is the C oracle (oracle/tilemix_oracle.h), linked as test code.
//
// Organisation (this program's own):
//   * every argument-validation expectation is one row of a table
//     (call, expected hipError_t), run before any HIP runtime call;
//   * closed forms of the score patterns are a table of (pattern, key count,
//     closed-form value) checked against the fp64 oracle;
//   * every GPU case is one Case record run by one function: all of a case's
//     device buffers come from one allocation (DeviceArena) in which each
//     buffer sits between guard bands that are verified after the case, and
//     inputs are proved unchanged by a hash of their bytes;
//   * --export-json writes one JSON object per GPU case (dense and routed) for
//     tests/native/fixture_check.py, the independent cross-check.
//
// The case lists, guard values, closed forms and the 1e-5 + 1e-4 |x| rule are
// data taken from the reference's test program (src/tests/tilemix_test.cu).
//
// Usage: tilemix_native [--cpu-only] [--export-json FILE] [--only TEXT] [--list]

#include "attention_fused.h"
#include "tilemix_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr int kIntMax = std::numeric_limits<int>::max();

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

void require(bool ok, const std::string& what) {
    if (!ok) fail(what);
}

void hip_check(hipError_t status, const char* what) {
    if (status != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(status));
}

// 64-bit FNV-1a over a byte range: inputs are hashed before the launches and
// after them to show that the library never writes them.
std::uint64_t fnv1a(const void* data, std::size_t bytes, std::uint64_t h = 0xcbf29ce484222325ull) {
    const auto* p = static_cast<const unsigned char*>(data);
    for (std::size_t i = 0; i < bytes; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
    return h;
}

// ------------------------------------------------------------- tolerance
struct ErrorStats {
    double max_abs = 0.0, max_rel = 0.0, rms = 0.0;
};

// Every element within atol + rtol |expected| (the reference's rule); the
// first element outside it ends the case with its index and both values.
template <class T>
ErrorStats within(const T* actual, const double* expected, std::size_t count, double atol, double rtol,
                  const std::string& label) {
    ErrorStats s;
    double squares = 0.0;
    for (std::size_t i = 0; i < count; ++i) {
        const double a = static_cast<double>(actual[i]), e = expected[i];
        const double err = std::fabs(a - e);
        if (!(std::isfinite(a) && std::isfinite(e) && err <= atol + rtol * std::fabs(e))) {
            std::ostringstream msg;
            msg.precision(17);
            msg << label << ": element " << i << " is " << a << ", expected " << e;
            fail(msg.str());
        }
        s.max_abs = std::max(s.max_abs, err);
        s.max_rel = std::max(s.max_rel, err / std::max(std::fabs(e), atol));
        squares += err * err;
    }
    s.rms = count ? std::sqrt(squares / static_cast<double>(count)) : 0.0;
    return s;
}

// ------------------------------------------------------------- CPU stage
struct Expectation {
    const char* name;
    std::function<hipError_t()> call;
    hipError_t want;
};

int run_validation_table() {
    static const __half one = __float2half(1.0f);
    static float o = 0.0f;
    static std::int8_t byte = 0;
    static __half scale_slot;
    static const std::uint64_t word = 0;
    const __half* x = &one;
    const float nan = std::numeric_limits<float>::quiet_NaN(), inf = std::numeric_limits<float>::infinity();
    auto attn = [](const __half* q, const __half* k, const __half* v, float* out, int m, int n, int d, float s,
                    const TileMixRouting& r = {}, const TileMixQuantized& z = {}) {
        return [=]() { return launch_fused_fp16_attention(q, k, v, out, m, n, d, s, nullptr, r, z); };
    };
    auto quant = [](const __half* q, const __half* k, std::int8_t* q8, std::int8_t* k8, __half* qs, __half* ks,
                    int m, int n, int d) {
        return [=]() { return quantize_tilemix_qk(q, k, q8, k8, qs, ks, m, n, d); };
    };
    const std::vector<Expectation> table = {
        {"attention: null Q", attn(nullptr, x, x, &o, 1, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: null K", attn(x, nullptr, x, &o, 1, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: null V", attn(x, x, nullptr, &o, 1, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: null O", attn(x, x, x, nullptr, 1, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: M = 0", attn(x, x, x, &o, 0, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: M < 0", attn(x, x, x, &o, -1, 1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: N = 0", attn(x, x, x, &o, 1, 0, 1, 1.0f), hipErrorInvalidValue},
        {"attention: N < 0", attn(x, x, x, &o, 1, -1, 1, 1.0f), hipErrorInvalidValue},
        {"attention: d = 0", attn(x, x, x, &o, 1, 1, 0, 1.0f), hipErrorInvalidValue},
        {"attention: d < 0", attn(x, x, x, &o, 1, 1, -1, 1.0f), hipErrorInvalidValue},
        {"attention: d = 129", attn(x, x, x, &o, 1, 1, 129, 1.0f), hipErrorNotSupported},
        {"attention: d = INT_MAX", attn(x, x, x, &o, 1, 1, kIntMax, 1.0f), hipErrorNotSupported},
        {"attention: NaN scale", attn(x, x, x, &o, 1, 1, 1, nan), hipErrorInvalidValue},
        {"attention: +inf scale", attn(x, x, x, &o, 1, 1, 1, inf), hipErrorInvalidValue},
        {"attention: -inf scale", attn(x, x, x, &o, 1, 1, 1, -inf), hipErrorInvalidValue},
        {"attention: partial quantized set", attn(x, x, x, &o, 1, 1, 1, 1.0f, {}, TileMixQuantized{&byte}),
         hipErrorInvalidValue},
        {"attention: key_tiles_per_group 0", attn(x, x, x, &o, 1, 1, 1, 1.0f, TileMixRouting{nullptr, 0, 0}),
         hipErrorInvalidValue},
        {"attention: key_tiles_per_group < 0", attn(x, x, x, &o, 1, 1, 1, 1.0f, TileMixRouting{nullptr, 0, -1}),
         hipErrorInvalidValue},
        {"attention: routing without quantized operands",
         attn(x, x, x, &o, 1, 1, 1, 1.0f, TileMixRouting{&word, 1, 1}), hipErrorInvalidValue},
        {"attention: null words with a count", attn(x, x, x, &o, 17, 2049, 1, 1.0f, TileMixRouting{nullptr, 1, 1}),
         hipErrorInvalidValue},
        {"attention: zero-length mask", attn(x, x, x, &o, 17, 2049, 1, 1.0f, TileMixRouting{&word, 0, 1}),
         hipErrorInvalidValue},
        {"attention: undersized mask", attn(x, x, x, &o, 17, 2049, 1, 1.0f, TileMixRouting{&word, 3, 1}),
         hipErrorInvalidValue},
        {"quantize: null Q", quant(nullptr, x, &byte, &byte, &scale_slot, &scale_slot, 1, 1, 1), hipErrorInvalidValue},
        {"quantize: null Q8", quant(x, x, nullptr, &byte, &scale_slot, &scale_slot, 1, 1, 1), hipErrorInvalidValue},
        {"quantize: null q_scales", quant(x, x, &byte, &byte, nullptr, &scale_slot, 1, 1, 1), hipErrorInvalidValue},
        {"quantize: M = 0", quant(x, x, &byte, &byte, &scale_slot, &scale_slot, 0, 1, 1), hipErrorInvalidValue},
        {"quantize: d = 129", quant(x, x, &byte, &byte, &scale_slot, &scale_slot, 1, 1, 129), hipErrorNotSupported},
    };
    for (const Expectation& e : table) {
        const hipError_t got = e.call();
        if (got != e.want)
            fail(std::string(e.name) + ": returned " + std::to_string(got) + ", expected " + std::to_string(e.want));
    }
    // Sizing helpers: compile-time values fixed by the reference's tests, and
    // the C-ABI mirrors at run time.
    static_assert(fused_fp16_shared_bytes(1) == 4608 && fused_fp16_shared_bytes(17) == 7168 &&
                  fused_fp16_shared_bytes(128) == 22528 && fused_fp16_shared_bytes(129) == 0);
    static_assert(kTileMixQQuantRows == 128 && kTileMixKQuantRows == 64);
    static_assert(tilemix_shared_bytes(128, true) == 28672 && tilemix_shared_bytes(17, true) == 8704);
    static_assert(tilemix_routing_word_count(17, 2048, 1) == 2 && tilemix_routing_word_count(17, 2049, 1) == 4 &&
                  tilemix_routing_word_count(17, 4097, 2) == 4 && tilemix_routing_word_count(17, 4097, 1) == 6 &&
                  tilemix_routing_word_count(17, kIntMax, kIntMax) == 2 && tilemix_routing_word_count(0, 1, 1) == 0 &&
                  tilemix_routing_word_count(1, 0, 1) == 0 && tilemix_routing_word_count(1, 1, 0) == 0);
    require(tilemix_shared_bytes_c(128, 1) == 28672 && tilemix_shared_bytes_c(17, 1) == 8704,
            "C-ABI shared-bytes mirror");
    require(tilemix_routing_word_count_c(17, 4097, 1) == 6 && tilemix_routing_word_count_c(1, 1, 0) == 0,
            "C-ABI routing word-count mirror");
    return static_cast<int>(table.size()) + 2;
}

std::vector<std::uint16_t> halves(std::size_t n) { return std::vector<std::uint16_t>(n); }

struct HostInputs {
    std::vector<std::uint16_t> q, k, v;
};

HostInputs make_inputs(int m, int n, int d, const char* pattern) {
    HostInputs in{halves(static_cast<std::size_t>(m) * d), halves(static_cast<std::size_t>(n) * d),
                  halves(static_cast<std::size_t>(n) * d)};
    require(tmo_make_inputs(m, n, d, pattern, in.q.data(), in.k.data(), in.v.data()) == 0,
            std::string("unknown input pattern ") + pattern);
    return in;
}

struct ClosedForm {
    const char* pattern;
    int keys;
    std::function<double(const HostInputs&)> value;
};

// The score patterns whose 17 query rows all have one closed-form output
// (d = 1), evaluated by the fp64 oracle.
int run_closed_forms() {
    const std::vector<ClosedForm> table = {
        {"rising", 65, [](const HostInputs&) {
             const double a = 32 * std::exp(-8.0), b = 32 * std::exp(-4.0);
             return (a - b + 2) / (a + b + 1);
         }},
        {"falling", 65, [](const HostInputs&) {
             const double b = 32 * std::exp(-4.0), c = std::exp(-8.0);
             return (32 - b + 2 * c) / (32 + b + c);
         }},
        {"alternating", 129, [](const HostInputs&) {
             const double a = 32 * std::exp(-10.0), b = 32 * std::exp(-6.0), c = 32 * std::exp(-12.0),
                          e = 32 * std::exp(-2.0);
             return (a - b + 2 * c - 2 * e + 3) / (a + b + c + e + 1);
         }},
        {"late-extreme", 65, [](const HostInputs&) { return 3.0; }},
        {"negative", 65, [](const HostInputs& in) {
             double sum = 0.0;
             for (std::uint16_t h : in.v) sum += tmo_half_to_float(h);
             return sum / static_cast<double>(in.v.size());
         }},
    };
    for (const ClosedForm& c : table) {
        const HostInputs in = make_inputs(17, c.keys, 1, c.pattern);
        std::vector<double> got(17);
        require(tmo_attention(in.q.data(), in.k.data(), in.v.data(), 17, c.keys, 1, got.data()) == 0,
                "oracle rejected a closed-form case");
        const std::vector<double> want(17, c.value(in));
        const ErrorStats s = within(got.data(), want.data(), 17, 1e-12, 1e-12, c.pattern);
        std::printf("PASS closed form %-12s max_abs_error=%.3g\n", c.pattern, s.max_abs);
    }
    return static_cast<int>(table.size());
}

// ------------------------------------------------------------- GPU stage
enum class Routes { none, fp16, int8, mixed };

const char* routes_name(Routes r) {
    switch (r) {
        case Routes::fp16: return "fp16";
        case Routes::int8: return "int8";
        case Routes::mixed: return "mixed";
        default: return "none";
    }
}

struct Case {
    int m, n, d;
    const char* pattern;
    Routes routes = Routes::none;
    int group = 1;              // key_tiles_per_group of the routing mask
    bool nonblocking = true;    // false: the default (null) stream

    std::string label() const {
        std::ostringstream s;
        s << "M=" << m << " N=" << n << " d=" << d << " pattern=" << pattern << " routes=" << routes_name(routes);
        if (routes != Routes::none) s << " g=" << group;
        s << " stream=" << (nonblocking ? "nonblocking" : "default");
        return s.str();
    }
};

std::vector<Case> gpu_cases() {
    std::vector<Case> cases;
    for (int d : {1, 15, 16, 17, 31, 32, 33, 49, 63, 64, 65, 81, 97, 113, 127, 128}) cases.push_back({3, 33, d, "random"});
    const Case dense[] = {{1, 1, 1, "random"}, {3, 5, 7, "random"}, {15, 31, 15, "random"}, {16, 32, 16, "random"},
                          {17, 33, 17, "random"}, {31, 63, 31, "random"}, {32, 64, 32, "random"},
                          {33, 65, 33, "random"}, {35, 67, 65, "random"}, {17, 65, 128, "random"},
                          {17, 1, 128, "random"}, {17, 33, 17, "random", Routes::none, 1, false},
                          {17, 65, 1, "rising"}, {17, 65, 1, "falling"}, {17, 129, 1, "alternating"},
                          {17, 65, 1, "late-extreme"}, {17, 33, 1, "negative"}, {17, 33, 17, "zeros"},
                          {17, 33, 17, "uniform"}, {17, 33, 17, "zero-v"}, {17, 65, 17, "constant-v"},
                          {2, 32, 17, "cancellation"}, {17, 33, 1, "large-dot"}, {3, 2051, 17, "random"},
                          {1, 4097, 128, "uniform"}};
    cases.insert(cases.end(), std::begin(dense), std::end(dense));
    struct RoutedShape { int m, n, d; const char* pattern; int group; };
    const RoutedShape routed[] = {{35, 67, 17, "random", 2}, {17, 2049, 5, "random", 1}, {17, 4099, 5, "random", 2},
                                  {35, 163, 17, "random", 3}, {17, 65, 17, "random", kIntMax},
                                  {129, 131, 17, "block-outliers", 1}, {17, 33, 128, "max-int8", 1},
                                  {3, 33, 64, "random", 1}, {3, 33, 128, "random", 1}};
    for (const RoutedShape& r : routed)
        for (Routes kind : {Routes::fp16, Routes::int8, Routes::mixed})
            cases.push_back({r.m, r.n, r.d, r.pattern, kind, r.group});
    return cases;
}

// One device allocation per case. Each buffer handed out is 256-byte aligned
// and sits between two 64-byte guard bands of a fixed byte pattern; after the
// case every band must still hold it (no write past or before any buffer).
class DeviceArena {
public:
    static constexpr std::size_t kBand = 64;
    static constexpr unsigned char kGuardByte = 0xA7;

    template <class T>
    T* take(std::size_t count) {
        Piece p{align(offset_ + kBand), count * sizeof(T)};
        offset_ = p.offset + p.bytes + kBand;
        pieces_.push_back(p);
        return reinterpret_cast<T*>(static_cast<std::uintptr_t>(p.offset));  // rebased by commit()
    }
    // Allocates the arena, fills every guard band, and rebases the pointers.
    template <class... Ptr>
    void commit(Ptr*&... ptrs) {
        offset_ = align(offset_);
        hip_check(hipMalloc(&base_, offset_), "hipMalloc");
        std::vector<unsigned char> fill(offset_, kGuardByte);
        hip_check(hipMemcpy(base_, fill.data(), offset_, hipMemcpyHostToDevice), "guard fill");
        (rebase(ptrs), ...);
    }
    void verify() const {
        std::vector<unsigned char> host(offset_);
        hip_check(hipMemcpy(host.data(), base_, offset_, hipMemcpyDeviceToHost), "guard read");
        for (const Piece& p : pieces_)
            for (std::size_t i = 1; i <= kBand; ++i)
                if (host[p.offset - i] != kGuardByte || host[p.offset + p.bytes + i - 1] != kGuardByte)
                    fail("a guard band next to a device buffer was overwritten");
    }
    ~DeviceArena() { (void)hipFree(base_); }

private:
    struct Piece { std::size_t offset, bytes; };
    static std::size_t align(std::size_t x) { return (x + 255) & ~std::size_t{255}; }
    template <class T>
    void rebase(T*& p) { p = reinterpret_cast<T*>(static_cast<unsigned char*>(base_) + reinterpret_cast<std::uintptr_t>(p)); }
    void* base_ = nullptr;
    std::size_t offset_ = 0;
    std::vector<Piece> pieces_;
};

template <class T>
void upload(T* dst, const std::vector<T>& src, hipStream_t s) {
    hip_check(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, s), "upload");
}
template <class T>
std::vector<T> download(const T* src, std::size_t count) {
    std::vector<T> host(count);
    hip_check(hipMemcpy(host.data(), src, count * sizeof(T), hipMemcpyDeviceToHost), "download");
    return host;
}

// Route code of a (16-row query tile, key-tile group) cell for a routed case.
// "mixed" sets 3 of every 7 cells along each diagonal-free line, so INT8 and
// FP16 cells both occur in every row with two or more groups, in every group
// column with two or more rows, and in each 64-group word of long rows.
bool cell_is_int8(Routes r, std::size_t row, std::size_t group) {
    if (r == Routes::int8) return true;
    if (r != Routes::mixed) return false;
    return (3 * (row % 7) + 5 * (group % 7) + 1) % 7 < 3;
}

struct RouteMask {
    std::vector<std::uint64_t> words;  // TileMixRouting packing
    std::vector<std::uint8_t> cells;   // expected trace: one code per 16x32 cell
};

RouteMask build_mask(const Case& c) {
    const std::size_t rows = (c.m - 1) / 16 + 1, key_tiles = (c.n - 1) / 32 + 1;
    const std::size_t groups = (key_tiles - 1) / static_cast<std::size_t>(c.group) + 1;
    const std::size_t per_row = (groups - 1) / 64 + 1;
    RouteMask mask{std::vector<std::uint64_t>(rows * per_row, 0), std::vector<std::uint8_t>(rows * key_tiles, 0)};
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t t = 0; t < key_tiles; ++t) {
            const std::size_t g = t / static_cast<std::size_t>(c.group);
            const bool int8 = cell_is_int8(c.routes, r, g);
            mask.cells[r * key_tiles + t] = int8;
            if (int8) mask.words[r * per_row + g / 64] |= std::uint64_t{1} << (g % 64);
        }
    require(mask.words.size() == tilemix_routing_word_count(c.m, c.n, c.group), "mask size != word count");
    return mask;
}

// A JSON Lines record writer: fields in call order, numbers at full precision.
class Record {
public:
    explicit Record(std::ostream& out) : out_(out) { out_.precision(std::numeric_limits<float>::max_digits10); }
    Record& field(const char* key, long long v) {
        key_(key) << v;
        return *this;
    }
    Record& field(const char* key, double v) {
        key_(key) << v;
        return *this;
    }
    Record& field(const char* key, const std::string& v) {
        key_(key) << '"' << v << '"';
        return *this;
    }
    template <class T, class F>
    Record& array(const char* key, const std::vector<T>& values, F convert) {
        key_(key) << '[';
        for (std::size_t i = 0; i < values.size(); ++i) out_ << (i ? "," : "") << convert(values[i]);
        out_ << ']';
        return *this;
    }
    void end() {
        out_ << "}\n";
        require(static_cast<bool>(out_), "could not write a JSON record");
    }

private:
    std::ostream& key_(const char* key) {
        out_ << (first_ ? "{" : ",") << '"' << key << "\":";
        first_ = false;
        return out_;
    }
    std::ostream& out_;
    bool first_ = true;
};

constexpr float kOutputGuard = -12345.25f;          // unwritten O elements
constexpr std::int32_t kDotGuard = 0x2468ace;      // score_dots of FP16 cells stay untouched
constexpr std::uint8_t kTraceFill = 0xa5;           // every trace byte is overwritten

void run_case(const Case& c, std::ostream* json) {
    const HostInputs in = make_inputs(c.m, c.n, c.d, c.pattern);
    const std::size_t nq = in.q.size(), nk = in.k.size();
    const bool routed = c.routes != Routes::none;
    const float scale = 1.0f / std::sqrt(static_cast<float>(c.d));
    const RouteMask mask = routed ? build_mask(c) : RouteMask{};

    DeviceArena arena;
    auto* q = arena.take<std::uint16_t>(nq);
    auto* k = arena.take<std::uint16_t>(nk);
    auto* v = arena.take<std::uint16_t>(nk);
    auto* o = arena.take<float>(nq);
    auto* o_plain = arena.take<float>(nq);
    auto* q8 = arena.take<std::int8_t>(nq);
    auto* k8 = arena.take<std::int8_t>(nk);
    auto* qs = arena.take<std::uint16_t>((c.m - 1) / 128 + 1);
    auto* ks = arena.take<std::uint16_t>((c.n - 1) / 64 + 1);
    auto* words = arena.take<std::uint64_t>(std::max<std::size_t>(mask.words.size(), 1));
    auto* trace = arena.take<std::uint8_t>(std::max<std::size_t>(mask.cells.size(), 1));
    auto* dots = arena.take<std::int32_t>(routed ? static_cast<std::size_t>(c.m) * c.n : 1);
    arena.commit(q, k, v, o, o_plain, q8, k8, qs, ks, words, trace, dots);

    hipStream_t stream = nullptr;
    if (c.nonblocking) hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "stream");
    struct StreamGuard { hipStream_t s; ~StreamGuard() { if (s) (void)hipStreamDestroy(s); } } guard{stream};
    upload(q, in.q, stream);
    upload(k, in.k, stream);
    upload(v, in.v, stream);
    upload(o, std::vector<float>(nq, kOutputGuard), stream);
    upload(o_plain, std::vector<float>(nq, kOutputGuard), stream);
    const std::uint64_t input_hash = fnv1a(in.v.data(), nk * 2, fnv1a(in.k.data(), nk * 2, fnv1a(in.q.data(), nq * 2)));
    const auto* hq = reinterpret_cast<const __half*>(q);
    const auto* hk = reinterpret_cast<const __half*>(k);
    const auto* hv = reinterpret_cast<const __half*>(v);

    std::vector<double> want(nq);
    std::vector<float> got;
    if (!routed) {
        hip_check(launch_fused_fp16_attention(hq, hk, hv, o, c.m, c.n, c.d, scale, stream), "attention");
        hip_check(hipStreamSynchronize(stream), "sync");
        got = download(o, nq);
        require(tmo_attention(in.q.data(), in.k.data(), in.v.data(), c.m, c.n, c.d, want.data()) == 0, "oracle");
    } else {
        upload(words, mask.words, stream);
        upload(trace, std::vector<std::uint8_t>(mask.cells.size(), kTraceFill), stream);
        upload(dots, std::vector<std::int32_t>(static_cast<std::size_t>(c.m) * c.n, kDotGuard), stream);
        hip_check(quantize_tilemix_qk(hq, hk, q8, k8, reinterpret_cast<__half*>(qs), reinterpret_cast<__half*>(ks),
                                      c.m, c.n, c.d, stream), "quantize");
        // The same inputs without routing: an all-FP16 mask must reproduce it bit for bit.
        hip_check(launch_fused_fp16_attention(hq, hk, hv, o_plain, c.m, c.n, c.d, scale, stream), "plain attention");
        const TileMixRouting routing{words, mask.words.size(), c.group, trace};
        const TileMixQuantized quantized{q8, k8, reinterpret_cast<const __half*>(qs),
                                         reinterpret_cast<const __half*>(ks), dots};
        hip_check(launch_fused_fp16_attention(hq, hk, hv, o, c.m, c.n, c.d, scale, stream, routing, quantized),
                  "routed attention");
        hip_check(hipStreamSynchronize(stream), "sync");
        got = download(o, nq);

        std::vector<std::int8_t> q8_ref(nq), k8_ref(nk);
        std::vector<std::uint16_t> qs_ref((c.m - 1) / 128 + 1), ks_ref((c.n - 1) / 64 + 1);
        tmo_quantize(in.q.data(), c.m, c.d, 128, q8_ref.data(), qs_ref.data());
        tmo_quantize(in.k.data(), c.n, c.d, 64, k8_ref.data(), ks_ref.data());
        require(download(q8, nq) == q8_ref && download(k8, nk) == k8_ref, "Q8/K8 differ from the oracle quantizer");
        require(download(qs, qs_ref.size()) == qs_ref && download(ks, ks_ref.size()) == ks_ref,
                "quantization scales differ from the oracle quantizer");
        require(download(trace, mask.cells.size()) == mask.cells, "routing trace differs from the mask");
        const std::vector<std::int32_t> d32 = download(dots, static_cast<std::size_t>(c.m) * c.n);
        const std::size_t key_tiles = (c.n - 1) / 32 + 1;
        for (int i = 0; i < c.m; ++i)
            for (int j = 0; j < c.n; ++j) {
                const bool int8 = mask.cells[(i / 16) * key_tiles + j / 32] != 0;
                const std::int32_t expect = int8 ? tmo_int8_dot(q8_ref.data(), k8_ref.data(), i, j, c.d) : kDotGuard;
                if (d32[static_cast<std::size_t>(i) * c.n + j] != expect)
                    fail("score_dots[" + std::to_string(i) + "][" + std::to_string(j) + "] is wrong");
            }
        if (c.routes == Routes::fp16) {
            const std::vector<float> plain = download(o_plain, nq);
            require(std::memcmp(plain.data(), got.data(), nq * sizeof(float)) == 0,
                    "an all-FP16 mask changed the un-routed output");
        }
        tmo_tilemix(in.q.data(), in.k.data(), in.v.data(), q8_ref.data(), k8_ref.data(), qs_ref.data(), ks_ref.data(),
                    mask.cells.data(), c.m, c.n, c.d, scale, 0, nullptr, 0, want.data());
    }
    const ErrorStats s = within(got.data(), want.data(), nq, 1e-5, 1e-4, c.label());
    arena.verify();
    const std::vector<std::uint16_t> q_after = download(q, nq), k_after = download(k, nk), v_after = download(v, nk);
    require(fnv1a(v_after.data(), nk * 2, fnv1a(k_after.data(), nk * 2, fnv1a(q_after.data(), nq * 2))) == input_hash,
            "the library wrote to Q, K or V");
    std::printf("PASS %s max_abs_error=%.3g max_rel_error=%.3g rms_error=%.3g\n", c.label().c_str(), s.max_abs,
                s.max_rel, s.rms);
    if (json) {
        Record r(*json);
        const auto as_float = [](std::uint16_t h) { return static_cast<double>(tmo_half_to_float(h)); };
        r.field("m", static_cast<long long>(c.m)).field("n", static_cast<long long>(c.n))
            .field("d", static_cast<long long>(c.d)).field("pattern", std::string(c.pattern))
            .array("q", in.q, as_float).array("k", in.k, as_float).array("v", in.v, as_float)
            .array("o", got, [](float f) { return static_cast<double>(f); })
            .field("scale", static_cast<double>(scale));
        if (routed) {
            std::string cells(mask.cells.size(), '0');
            for (std::size_t i = 0; i < cells.size(); ++i) cells[i] = mask.cells[i] ? '1' : '0';
            r.field("routes", cells);
        }
        r.end();
    }
}

struct Options {
    bool cpu_only = false, list = false;
    std::string json_path, only;
};

Options parse(int argc, char** argv) {
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--cpu-only") o.cpu_only = true;
        else if (a == "--list") o.list = true;
        else if (a == "--export-json" && i + 1 < argc) o.json_path = argv[++i];
        else if (a == "--only" && i + 1 < argc) o.only = argv[++i];
        else throw std::invalid_argument("usage: tilemix_native [--cpu-only] [--export-json FILE] [--only TEXT] [--list]");
    }
    return o;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const Options opt = parse(argc, argv);
        std::vector<Case> cases = gpu_cases();
        if (!opt.only.empty())
            cases.erase(std::remove_if(cases.begin(), cases.end(),
                                       [&](const Case& c) { return c.label().find(opt.only) == std::string::npos; }),
                        cases.end());
        if (opt.list) {
            for (const Case& c : cases) std::puts(c.label().c_str());
            return 0;
        }
        const int validated = run_validation_table();
        std::printf("PASS API validation: %d expectations, no HIP runtime call made\n", validated);
        const int closed = run_closed_forms();
        std::printf("PASS closed forms: %d patterns against the fp64 oracle\n", closed);
        if (opt.cpu_only) return 0;

        hipDeviceProp_t props{};
        int device = 0;
        hip_check(hipGetDevice(&device), "hipGetDevice");
        hip_check(hipGetDeviceProperties(&props, device), "hipGetDeviceProperties");
        std::printf("device %d: %s (%s)\n", device, props.name, props.gcnArchName);
        std::ofstream json;
        if (!opt.json_path.empty()) {
            json.open(opt.json_path);
            require(static_cast<bool>(json), "could not open " + opt.json_path);
        }
        int dense = 0, routed = 0;
        for (const Case& c : cases) {
            run_case(c, json.is_open() ? &json : nullptr);
            (c.routes == Routes::none ? dense : routed) += 1;
        }
        std::printf("PASS GPU cases: %d dense + %d routed, all within 1e-5 + 1e-4|x| of the fp64 oracle\n", dense,
                    routed);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: %s\n", e.what());
        return 1;
    }
}
