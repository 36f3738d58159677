// Device-side producer of TileMix routing masks for gfx950.
//
// The reference builds its masks on the host: the test packer
// (src/tests/tilemix_test.cu:432-448) and the demo's constant words
// (src/main.cu:48); the word format is include/attention_fused.h:34-52. Here
// the masks are produced on the GPU in two stages:
//
//  * builders write one code per coarse tile (tile_rows x tile_keys, whole
//    16 x 32 routing cells): 0 FP16, 1 INT8, 2 skip, laid out
//    [heads][tiles_q][tiles_k];
//  * the packer turns tile codes into route / skip words
//    ([heads][ceil(M/16)][words_per_row] uint64, one bit per group of
//    key_tiles_per_group 32-key tiles).
//
// Random builders draw from a counter-based generator (splitmix64 of the
// seed and the tile's linear index), so the result depends only on
// (seed, head, tile) and a host restatement reproduces it bit for bit. The
// importance router ranks tiles by the |q.k| bound d * amax_Q * amax_K with
// an exact per-head radix select (ties broken by tile index).

#include "tilemix_capi.h"
#include "tilemix_device.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

namespace tilemix {
namespace {

constexpr int kCellRows = 16;
constexpr int kCellKeys = 32;
constexpr std::uint8_t kFp16 = TILEMIX_ROUTE_FP16;
constexpr std::uint8_t kInt8 = TILEMIX_ROUTE_INT8;
constexpr std::uint8_t kSkip = TILEMIX_ROUTE_SKIP;
constexpr int kSelectThreads = 1024;
constexpr int kMaxSelectEntries = 16384;  // tiles_q + tiles_k kept in LDS by the importance select

__host__ __device__ inline std::uint64_t splitmix64(std::uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Uniform in [0, 1) with 24 random bits (exact in fp32) for counter `index`
// of stream `salt` (0 = tile draws, 1 = the forced-FP16 column of the
// three-way builder).
__device__ inline float uniform24(std::uint64_t seed, std::uint64_t index, std::uint64_t salt) {
    const std::uint64_t h = splitmix64(seed ^ splitmix64(2 * index + salt));
    return static_cast<float>(h >> 40) * (1.0f / 16777216.0f);
}

__global__ void bernoulli_kernel(std::uint8_t* codes, std::int64_t total, float p_int8, std::uint64_t seed) {
    const std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    codes[t] = uniform24(seed, static_cast<std::uint64_t>(t), 0) < p_int8 ? kInt8 : kFp16;
}

// Tile (i, j) of a square causal problem: skipped when its first key is past
// the tile's last query row, FP16 for the fp16_band key tiles ending at the
// diagonal tile, otherwise INT8 with probability p_int8.
__global__ void causal_band_kernel(std::uint8_t* codes, int heads, int tiles_q, int tiles_k, int tile_rows,
                                   int tile_keys, int fp16_band, float p_int8, std::uint64_t seed) {
    const std::int64_t total = static_cast<std::int64_t>(heads) * tiles_q * tiles_k;
    const std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int j = static_cast<int>(t % tiles_k);
    const int i = static_cast<int>((t / tiles_k) % tiles_q);
    const std::int64_t last_visible = (static_cast<std::int64_t>(i) * tile_rows + tile_rows - 1) / tile_keys;
    std::uint8_t code;
    if (j > last_visible) code = kSkip;
    else if (last_visible - j < fp16_band) code = kFp16;
    else code = uniform24(seed, static_cast<std::uint64_t>(t), 0) < p_int8 ? kInt8 : kFp16;
    codes[t] = code;
}

// One thread per (head, tile row): skip / INT8 / FP16 with probabilities
// p_skip / p_int8 / rest; a row left entirely skipped gets one tile (column
// from salt-1 draw of the row) forced FP16.
__global__ void three_way_kernel(std::uint8_t* codes, int rows, int tiles_k, float p_skip, float p_int8,
                                 std::uint64_t seed) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    std::uint8_t* out = codes + static_cast<std::int64_t>(row) * tiles_k;
    bool all_skip = true;
    for (int j = 0; j < tiles_k; ++j) {
        const float u = uniform24(seed, static_cast<std::uint64_t>(row) * tiles_k + j, 0);
        const std::uint8_t code = u < p_skip ? kSkip : (u < p_skip + p_int8 ? kInt8 : kFp16);
        all_skip = all_skip && code == kSkip;
        out[j] = code;
    }
    if (all_skip) {
        const std::uint64_t h = splitmix64(seed ^ splitmix64(2 * static_cast<std::uint64_t>(row) + 1));
        out[h % static_cast<std::uint64_t>(tiles_k)] = kFp16;
    }
}

// Absolute maximum of each tile row block of Q (blockIdx.x < tiles_q) and
// each key block of K (the rest), per head (blockIdx.y): amax[head][tiles_q +
// tiles_k].
__global__ __launch_bounds__(256) void tile_absmax_kernel(const std::uint16_t* Q, const std::uint16_t* K, int M,
                                                          int N, int d, std::int64_t q_stride,
                                                          std::int64_t k_stride, int tiles_q, int tiles_k,
                                                          int tile_rows, int tile_keys, float* amax) {
    __shared__ float partial[256 / kWave];
    const int head = blockIdx.y;
    const bool is_q = static_cast<int>(blockIdx.x) < tiles_q;
    const int block = is_q ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) - tiles_q;
    const int span = is_q ? tile_rows : tile_keys;
    const int rows = is_q ? M : N;
    const int first = block * span;
    const int last = min(rows, first + span);
    const std::uint16_t* x = (is_q ? Q + head * q_stride : K + head * k_stride) + static_cast<std::int64_t>(first) * d;
    const std::int64_t count = static_cast<std::int64_t>(last - first) * d;
    float m = 0.0f;
    for (std::int64_t e = threadIdx.x; e < count; e += 256) m = fmaxf(m, fabsf(half_bits_to_float(x[e])));
    m = wave_max(m);
    if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
        amax[static_cast<std::int64_t>(head) * (tiles_q + tiles_k) + blockIdx.x] = m;
    }
}

// One workgroup per head: the `count` tiles with the largest amax_Q(i) *
// amax_K(j) (exact in fp32: both are fp16 magnitudes; the factor d does not
// change the order) become FP16, ties going to the lower tile index; the
// rest INT8. Radix select on the float bits (non-negative, so integer order
// is value order), then one pass in index order that ranks the ties.
__global__ __launch_bounds__(kSelectThreads) void importance_select_kernel(const float* amax, int tiles_q,
                                                                            int tiles_k, std::int64_t count,
                                                                            std::uint8_t* codes) {
    extern __shared__ float factors[];  // tiles_q + tiles_k
    __shared__ unsigned histogram[256];
    __shared__ unsigned scan[kSelectThreads];
    __shared__ unsigned chosen_digit;
    __shared__ unsigned long long still_needed;
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    const int entries = tiles_q + tiles_k;
    for (int e = t; e < entries; e += kSelectThreads)
        factors[e] = amax[static_cast<std::int64_t>(head) * entries + e];
    const std::int64_t total = static_cast<std::int64_t>(tiles_q) * tiles_k;
    std::uint8_t* out = codes + static_cast<std::int64_t>(head) * total;
    auto key_of = [&](std::int64_t index) {
        const float e = factors[index / tiles_k] * factors[tiles_q + index % tiles_k];
        return __float_as_uint(e);
    };
    if (t == 0) still_needed = static_cast<unsigned long long>(count);
    __syncthreads();
    if (count <= 0 || count >= total) {
        const std::uint8_t code = count <= 0 ? kInt8 : kFp16;
        for (std::int64_t e = t; e < total; e += kSelectThreads) out[e] = code;
        return;
    }
    unsigned prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = t; b < 256; b += kSelectThreads) histogram[b] = 0;
        __syncthreads();
        for (std::int64_t e = t; e < total; e += kSelectThreads) {
            const unsigned key = key_of(e);
            if ((key & mask) == prefix) atomicAdd(&histogram[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (t == 0) {
            // Largest digit first: the digit whose bin holds the still-needed rank.
            unsigned long long above = 0;
            unsigned digit = 0;
            for (int b = 255; b >= 0; --b) {
                if (above + histogram[b] >= still_needed) {
                    digit = static_cast<unsigned>(b);
                    break;
                }
                above += histogram[b];
            }
            chosen_digit = digit;
            still_needed -= above;
        }
        __syncthreads();
        prefix |= chosen_digit << shift;
        mask |= 255u << shift;
    }
    // prefix = the count-th largest key; still_needed = how many of the keys
    // equal to it are FP16 (the lowest indices).
    const unsigned long long ties = still_needed;
    unsigned long long ties_before = 0;
    for (std::int64_t base = 0; base < total; base += kSelectThreads) {
        const std::int64_t e = base + t;
        const unsigned key = e < total ? key_of(e) : 0u;
        const unsigned equal = (e < total && key == prefix) ? 1u : 0u;
        scan[t] = equal;
        __syncthreads();
        // Inclusive scan (Hillis-Steele) of the tie flags in index order.
        for (int offset = 1; offset < kSelectThreads; offset <<= 1) {
            const unsigned add = t >= offset ? scan[t - offset] : 0u;
            __syncthreads();
            scan[t] += add;
            __syncthreads();
        }
        if (e < total) {
            const unsigned long long rank = ties_before + scan[t] - equal;
            out[e] = (key > prefix || (equal && rank < ties)) ? kFp16 : kInt8;
        }
        ties_before += scan[kSelectThreads - 1];
        __syncthreads();
    }
}

// One thread per output word: bit b of word w of query tile qt is group
// 64w + b, whose key tiles lie in coarse tile (kt * 32) / tile_keys.
__global__ void pack_kernel(const std::uint8_t* codes, int heads, int q_tiles16, int words_per_row, int groups,
                            int key_tiles_per_group, int tiles_q, int tiles_k, int tile_rows, int tile_keys,
                            std::uint64_t* route_words, std::uint64_t* skip_words) {
    const std::int64_t total = static_cast<std::int64_t>(heads) * q_tiles16 * words_per_row;
    const std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int w = static_cast<int>(t % words_per_row);
    const int qt = static_cast<int>((t / words_per_row) % q_tiles16);
    const std::int64_t head = t / (static_cast<std::int64_t>(words_per_row) * q_tiles16);
    const int i = qt * kCellRows / tile_rows;
    const std::uint8_t* row = codes + (head * tiles_q + i) * tiles_k;
    std::uint64_t route = 0, skip = 0;
    for (int b = 0; b < 64; ++b) {
        const int group = 64 * w + b;
        if (group >= groups) break;
        const std::int64_t kt = static_cast<std::int64_t>(group) * key_tiles_per_group;
        const std::uint8_t code = row[kt * kCellKeys / tile_keys];
        route |= static_cast<std::uint64_t>(code == kInt8) << b;
        skip |= static_cast<std::uint64_t>(code == kSkip) << b;
    }
    route_words[t] = route;
    skip_words[t] = skip;
}

unsigned blocks_for(std::int64_t items, int threads) {
    return static_cast<unsigned>((items + threads - 1) / threads);
}

bool tile_shape_ok(int tile_rows, int tile_keys) {
    return tile_rows > 0 && tile_keys > 0 && tile_rows % kCellRows == 0 && tile_keys % kCellKeys == 0;
}

bool probability_ok(float p) { return std::isfinite(p) && p >= 0.0f && p <= 1.0f; }

std::int64_t tile_count(int heads, int M, int N, int tile_rows, int tile_keys) {
    return static_cast<std::int64_t>(heads) * ((M - 1) / tile_rows + 1) * ((N - 1) / tile_keys + 1);
}

bool grid_ok(std::int64_t items, int threads) { return blocks_for(items, threads) <= 0x7fffffffu && items > 0; }

}  // namespace
}  // namespace tilemix

extern "C" int tilemix_routes_from_tiles(const std::uint8_t* tile_codes, int heads, int M, int N, int tile_rows,
                                         int tile_keys, int key_tiles_per_group, std::uint64_t* route_words,
                                         std::uint64_t* skip_words, void* stream) {
    using namespace tilemix;
    if (!tile_codes || !route_words || !skip_words || heads <= 0 || M <= 0 || N <= 0 || key_tiles_per_group <= 0 ||
        !tile_shape_ok(tile_rows, tile_keys) || (tile_keys / kCellKeys) % key_tiles_per_group != 0)
        return hipErrorInvalidValue;
    const int q_tiles16 = (M - 1) / kCellRows + 1;
    const int key_tiles32 = (N - 1) / kCellKeys + 1;
    const int groups = (key_tiles32 - 1) / key_tiles_per_group + 1;
    const int words_per_row = (groups - 1) / 64 + 1;
    const std::int64_t words = static_cast<std::int64_t>(heads) * q_tiles16 * words_per_row;
    if (!grid_ok(words, 256)) return hipErrorInvalidConfiguration;
    const int tiles_q = (M - 1) / tile_rows + 1, tiles_k = (N - 1) / tile_keys + 1;
    pack_kernel<<<blocks_for(words, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        tile_codes, heads, q_tiles16, words_per_row, groups, key_tiles_per_group, tiles_q, tiles_k, tile_rows,
        tile_keys, route_words, skip_words);
    return hipGetLastError();
}

extern "C" int tilemix_tiles_bernoulli(std::uint8_t* tile_codes, int heads, int M, int N, int tile_rows,
                                       int tile_keys, float p_int8, std::uint64_t seed, void* stream) {
    using namespace tilemix;
    if (!tile_codes || heads <= 0 || M <= 0 || N <= 0 || !tile_shape_ok(tile_rows, tile_keys) ||
        !probability_ok(p_int8))
        return hipErrorInvalidValue;
    const std::int64_t total = tile_count(heads, M, N, tile_rows, tile_keys);
    if (!grid_ok(total, 256)) return hipErrorInvalidConfiguration;
    bernoulli_kernel<<<blocks_for(total, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(tile_codes, total,
                                                                                            p_int8, seed);
    return hipGetLastError();
}

extern "C" int tilemix_tiles_causal_band(std::uint8_t* tile_codes, int heads, int S, int tile_rows, int tile_keys,
                                         int fp16_band, float p_int8, std::uint64_t seed, void* stream) {
    using namespace tilemix;
    if (!tile_codes || heads <= 0 || S <= 0 || !tile_shape_ok(tile_rows, tile_keys) || fp16_band < 0 ||
        !probability_ok(p_int8))
        return hipErrorInvalidValue;
    const int tiles_q = (S - 1) / tile_rows + 1, tiles_k = (S - 1) / tile_keys + 1;
    const std::int64_t total = static_cast<std::int64_t>(heads) * tiles_q * tiles_k;
    if (!grid_ok(total, 256)) return hipErrorInvalidConfiguration;
    causal_band_kernel<<<blocks_for(total, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        tile_codes, heads, tiles_q, tiles_k, tile_rows, tile_keys, fp16_band, p_int8, seed);
    return hipGetLastError();
}

extern "C" int tilemix_tiles_three_way(std::uint8_t* tile_codes, int heads, int M, int N, int tile_rows,
                                       int tile_keys, float p_skip, float p_int8, std::uint64_t seed,
                                       void* stream) {
    using namespace tilemix;
    if (!tile_codes || heads <= 0 || M <= 0 || N <= 0 || !tile_shape_ok(tile_rows, tile_keys) ||
        !probability_ok(p_skip) || !probability_ok(p_int8) || p_skip + p_int8 > 1.0f)
        return hipErrorInvalidValue;
    const int tiles_q = (M - 1) / tile_rows + 1, tiles_k = (N - 1) / tile_keys + 1;
    const std::int64_t rows = static_cast<std::int64_t>(heads) * tiles_q;
    if (rows > 0x7fffffff || !grid_ok(rows, 256)) return hipErrorInvalidConfiguration;
    three_way_kernel<<<blocks_for(rows, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        tile_codes, static_cast<int>(rows), tiles_k, p_skip, p_int8, seed);
    return hipGetLastError();
}

extern "C" std::size_t tilemix_importance_workspace_bytes(int heads, int M, int N, int tile_rows, int tile_keys) {
    if (heads <= 0 || M <= 0 || N <= 0 || tile_rows <= 0 || tile_keys <= 0) return 0;
    const std::size_t entries = static_cast<std::size_t>((M - 1) / tile_rows + 1) + ((N - 1) / tile_keys + 1);
    return static_cast<std::size_t>(heads) * entries * sizeof(float);
}

// Scratch of tilemix_tiles_importance_noalloc: the per-tile maxima of up to
// kImportanceScratchFloats / (tiles_q + tiles_k) heads. One copy per GPU,
// held until the process ends; every call on a GPU shares it, so calls that
// overlap on one GPU race.
static constexpr std::size_t kImportanceScratchFloats = std::size_t{1} << 18;  // 1 MiB
static __device__ __align__(256) float scratch[kImportanceScratchFloats];

namespace tilemix {
namespace {

// Device address of `scratch` on the current device, looked up once per
// device with that device current (in host code the array's name is only a
// host-side stand-in, not a device address).
hipError_t scratch_address(float** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex lock;
    static float* address[kMaxDevices] = {};
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return status;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(lock);
    if (!address[device]) {
        void* ptr = nullptr;
        status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (status != hipSuccess) return status;
        address[device] = static_cast<float*>(ptr);
    }
    *out = address[device];
    return hipSuccess;
}

// Argument checks shared by both importance entry points, in two groups so
// that each entry point can keep its order (no runtime call): values first
// (InvalidValue), limits after the caller's own buffer-size check.
bool importance_values_ok(const std::uint16_t* Q, const std::uint16_t* K, int heads, int M, int N, int d,
                          std::int64_t q_head_stride, std::int64_t k_head_stride, int tile_rows, int tile_keys,
                          float fp16_fraction, const std::uint8_t* tile_codes) {
    if (!Q || !K || !tile_codes || heads <= 0 || M <= 0 || N <= 0 || d <= 0 ||
        !tile_shape_ok(tile_rows, tile_keys) || !probability_ok(fp16_fraction))
        return false;
    return heads == 1 || (q_head_stride >= static_cast<std::int64_t>(M) * d &&
                          k_head_stride >= static_cast<std::int64_t>(N) * d);
}

hipError_t importance_limits(int heads, int M, int N, int tile_rows, int tile_keys) {
    const int tiles_q = (M - 1) / tile_rows + 1, tiles_k = (N - 1) / tile_keys + 1;
    if (tiles_q + tiles_k > kMaxSelectEntries) return hipErrorNotSupported;
    if (heads > 65535) return hipErrorInvalidConfiguration;
    return hipSuccess;
}

// Tile maxima into `workspace`, then the per-head select into tile_codes.
hipError_t launch_importance(const std::uint16_t* Q, const std::uint16_t* K, int heads, int M, int N, int d,
                             std::int64_t q_head_stride, std::int64_t k_head_stride, int tile_rows, int tile_keys,
                             float fp16_fraction, float* workspace, std::uint8_t* tile_codes, hipStream_t s) {
    const int tiles_q = (M - 1) / tile_rows + 1, tiles_k = (N - 1) / tile_keys + 1;
    const std::int64_t total = static_cast<std::int64_t>(tiles_q) * tiles_k;
    // The number of FP16 tiles: fp16_fraction * total rounded half to even.
    const std::int64_t count = static_cast<std::int64_t>(std::nearbyint(static_cast<double>(fp16_fraction) * total));
    const std::int64_t qs = heads > 1 ? q_head_stride : static_cast<std::int64_t>(M) * d;
    const std::int64_t ks = heads > 1 ? k_head_stride : static_cast<std::int64_t>(N) * d;
    tile_absmax_kernel<<<dim3(static_cast<unsigned>(tiles_q + tiles_k), static_cast<unsigned>(heads)), 256, 0, s>>>(
        Q, K, M, N, d, qs, ks, tiles_q, tiles_k, tile_rows, tile_keys, workspace);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    importance_select_kernel<<<static_cast<unsigned>(heads), kSelectThreads,
                               static_cast<std::size_t>(tiles_q + tiles_k) * sizeof(float), s>>>(
        workspace, tiles_q, tiles_k, count, tile_codes);
    return hipGetLastError();
}

}  // namespace
}  // namespace tilemix

extern "C" int tilemix_tiles_importance(const std::uint16_t* Q, const std::uint16_t* K, int heads, int M, int N,
                                        int d, std::int64_t q_head_stride, std::int64_t k_head_stride,
                                        int tile_rows, int tile_keys, float fp16_fraction, float* workspace,
                                        std::size_t workspace_bytes, std::uint8_t* tile_codes, void* stream) {
    using namespace tilemix;
    if (!workspace || !importance_values_ok(Q, K, heads, M, N, d, q_head_stride, k_head_stride, tile_rows,
                                            tile_keys, fp16_fraction, tile_codes))
        return hipErrorInvalidValue;
    if (workspace_bytes < tilemix_importance_workspace_bytes(heads, M, N, tile_rows, tile_keys))
        return hipErrorInvalidValue;
    const hipError_t limits = importance_limits(heads, M, N, tile_rows, tile_keys);
    if (limits != hipSuccess) return limits;
    return launch_importance(Q, K, heads, M, N, d, q_head_stride, k_head_stride, tile_rows, tile_keys,
                             fp16_fraction, workspace, tile_codes, static_cast<hipStream_t>(stream));
}

extern "C" std::size_t tilemix_importance_noalloc_max_bytes(void) {
    return kImportanceScratchFloats * sizeof(float);
}

extern "C" int tilemix_tiles_importance_noalloc(const std::uint16_t* Q, const std::uint16_t* K, int heads, int M,
                                                int N, int d, std::int64_t q_head_stride,
                                                std::int64_t k_head_stride, int tile_rows, int tile_keys,
                                                float fp16_fraction, std::uint8_t* tile_codes, void* stream) {
    using namespace tilemix;
    if (!importance_values_ok(Q, K, heads, M, N, d, q_head_stride, k_head_stride, tile_rows, tile_keys,
                              fp16_fraction, tile_codes))
        return hipErrorInvalidValue;
    // More tile maxima than the fixed scratch holds.
    if (tilemix_importance_workspace_bytes(heads, M, N, tile_rows, tile_keys) > tilemix_importance_noalloc_max_bytes())
        return hipErrorInvalidValue;
    const hipError_t limits = importance_limits(heads, M, N, tile_rows, tile_keys);
    if (limits != hipSuccess) return limits;
    float* workspace = nullptr;
    const hipError_t found = scratch_address(&workspace);
    if (found != hipSuccess) return found;
    // The tile-maxima kernel writes every entry the select reads, so the
    // previous call's contents need no clearing.
    return launch_importance(Q, K, heads, M, N, d, q_head_stride, k_head_stride, tile_rows, tile_keys,
                             fp16_fraction, workspace, tile_codes, static_cast<hipStream_t>(stream));
}
