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
// tiles_k]. NaN elements are passed over, as fmaxf does. kVector (d % 8 == 0,
// 16-byte aligned heads): 16-byte loads and the maximum over fp16 bit
// patterns with the sign cleared (unsigned order is value order for them;
// NaN patterns sort above +inf, so a maximum above 0x7c00 sends the block
// through a second pass that leaves NaNs out).
template <bool kVector>
__global__ __launch_bounds__(256) void tile_absmax_kernel(const std::uint16_t* Q, const std::uint16_t* K, int M,
                                                          int N, int d, std::int64_t q_stride,
                                                          std::int64_t k_stride, int tiles_q, int tiles_k,
                                                          int tile_rows, int tile_keys, float* amax) {
    __shared__ float partial[256 / kWave];
    __shared__ unsigned partial_bits[256 / kWave];
    const int head = blockIdx.y;
    const bool is_q = static_cast<int>(blockIdx.x) < tiles_q;
    const int block = is_q ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) - tiles_q;
    const int span = is_q ? tile_rows : tile_keys;
    const int rows = is_q ? M : N;
    const int first = block * span;
    const int last = min(rows, first + span);
    const std::uint16_t* x = (is_q ? Q + head * q_stride : K + head * k_stride) + static_cast<std::int64_t>(first) * d;
    const std::int64_t count = static_cast<std::int64_t>(last - first) * d;
    const std::int64_t slot = static_cast<std::int64_t>(head) * (tiles_q + tiles_k) + blockIdx.x;
    if constexpr (kVector) {
        // Eight 16-byte loads in flight per thread, then their maximum.
        constexpr int kLoads = 8;
        const std::int64_t chunks = count / 8;
        unsigned top = 0;
        for (std::int64_t base = threadIdx.x; base < chunks; base += kLoads * 256) {
            uint4v v[kLoads];
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                const std::int64_t c = base + u * 256;
                v[u] = c < chunks ? *reinterpret_cast<const uint4v*>(x + 8 * c) : uint4v{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < kLoads; ++u)
#pragma unroll
                for (int w = 0; w < 4; ++w) top = max_u16x2(top, v[u][w] & 0x7fff7fffu);
        }
        unsigned bits = wave_max_bits(max(top & 0xffffu, top >> 16));
        if ((threadIdx.x & (kWave - 1)) == 0) partial_bits[threadIdx.x / kWave] = bits;
        __syncthreads();
        bits = max(max(partial_bits[0], partial_bits[1]), max(partial_bits[2], partial_bits[3]));
        if (bits > 0x7c00u) {
            // A NaN in the block: the maximum over the other elements.
            unsigned clean = 0;
            for (std::int64_t e = threadIdx.x; e < count; e += 256) {
                const unsigned h = x[e] & 0x7fffu;
                clean = h <= 0x7c00u ? max(clean, h) : clean;
            }
            clean = wave_max_bits(clean);
            __syncthreads();
            if ((threadIdx.x & (kWave - 1)) == 0) partial_bits[threadIdx.x / kWave] = clean;
            __syncthreads();
            bits = max(max(partial_bits[0], partial_bits[1]), max(partial_bits[2], partial_bits[3]));
        }
        if (threadIdx.x == 0) amax[slot] = half_bits_to_float(static_cast<std::uint16_t>(bits));
    } else {
        float m = 0.0f;
        for (std::int64_t e = threadIdx.x; e < count; e += 256) m = fmaxf(m, fabsf(half_bits_to_float(x[e])));
        m = wave_max(m);
        if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = m;
        __syncthreads();
        if (threadIdx.x == 0) amax[slot] = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
    }
}

// One workgroup per head: the `count` tiles with the largest amax_Q(i) *
// amax_K(j) (exact in fp32: both are fp16 magnitudes; the factor d does not
// change the order) become FP16, ties going to the lower tile index; the
// rest INT8. The keys are the products' float bits (non-negative, so integer
// order is value order) minus the head's smallest key; a radix select over
// the bits of (largest - smallest), at most 11 bits a pass (three passes
// cover any range), finds the count-th largest key with one histogram of
// 2048 bins and a block-wide scan over its bins per pass. Then one pass in
// index order sets the codes, ranking the ties with wave ballots only when
// some of the keys equal to the selected one stay INT8.
//
// kKeys > 0 (a head of at most 1024 kKeys tiles): wave w holds tiles
// [64 kKeys w, 64 kKeys (w + 1)) in registers, tile 64 kKeys w + 64 u + lane
// in keys[u], so a pass reads no memory, the code stores of a wave are
// contiguous, and the ties before a tile are those of earlier waves plus the
// wave's own earlier slots and lanes. Tiles past the end take the smallest
// key, which leaves the selection unchanged (count < total, and their indices
// sort them after every valid tile of equal key); they are never stored.
// kKeys == 0: thread t recomputes tiles t, t + 1024, ... each pass, its (row,
// column) advancing by a fixed step, and ties are ranked 1024 tiles at a time.
template <int kKeys>
__global__ __launch_bounds__(kSelectThreads) void importance_select_kernel(const float* amax, int tiles_q,
                                                                            int tiles_k, std::int64_t count,
                                                                            std::uint8_t* codes) {
    constexpr int kWaves = kSelectThreads / kWave;
    constexpr int kDigitBits = 11;
    constexpr int kBins = 1 << kDigitBits;
    static_assert(kBins == 2 * kSelectThreads, "two bins per thread in the digit scan");
    extern __shared__ float factors[];  // tiles_q + tiles_k
    __shared__ unsigned histogram[kBins];
    __shared__ unsigned wave_low[kWaves], wave_high[kWaves];
    __shared__ unsigned chosen_digit, still_needed, equal_keys;
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    const int wave = t / kWave, lane = t & (kWave - 1);
    const int entries = tiles_q + tiles_k;
    for (int e = t; e < entries; e += kSelectThreads)
        factors[e] = amax[static_cast<std::int64_t>(head) * entries + e];
    // At most 8192 * 8192 tiles (tiles_q + tiles_k <= 16384): counts fit 32 bits.
    const std::int64_t total = static_cast<std::int64_t>(tiles_q) * tiles_k;
    std::uint8_t* out = codes + static_cast<std::int64_t>(head) * total;
    if (t == 0) still_needed = static_cast<unsigned>(count);
    __syncthreads();
    if (count <= 0 || count >= total) {
        const std::uint8_t code = count <= 0 ? kInt8 : kFp16;
        for (std::int64_t e = t; e < total; e += kSelectThreads) out[e] = code;
        return;
    }
    auto key_at = [&](int row, int col) { return __float_as_uint(factors[row] * factors[tiles_q + col]); };
    // The first tile this thread visits and the fixed step between its tiles.
    constexpr int kStep = kKeys > 0 ? kWave : kSelectThreads;
    const int first = kKeys > 0 ? wave * kWave * kKeys + lane : t;
    const int row0 = first / tiles_k, col0 = first % tiles_k;
    const int row_step = kStep / tiles_k, col_step = kStep % tiles_k;
    auto advance = [&](int& row, int& col) {
        row += row_step;
        col += col_step;
        if (col >= tiles_k) {
            col -= tiles_k;
            ++row;
        }
    };
    // kKeys > 0: total <= 1024 kKeys, so `remaining` (tiles from this
    // thread's first on) fits an int; slot u is in range when 64 u < remaining.
    // in_range() hides the value from the compiler so that it recomputes the
    // comparisons where they are needed instead of holding their lane masks.
    const int remaining = kKeys > 0 ? static_cast<int>(total) - first : 0;
    auto in_range = [&]() {
        int r = remaining;
        asm volatile("" : "+v"(r));
        return r;
    };
    unsigned keys[kKeys > 0 ? kKeys : 1];
    unsigned low = ~0u, high = 0u;
    if constexpr (kKeys > 0) {
        // (row, column) step from slot to slot; the empty asm keeps the
        // compiler from re-deriving every slot's column from the first.
        const int r = in_range();
        int row = row0, col = col0;
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            keys[u] = key_at(min(row, tiles_q - 1), col);
            const bool valid = u * kWave < r;
            low = valid ? min(low, keys[u]) : low;
            high = valid ? max(high, keys[u]) : high;
            advance(row, col);
            asm volatile("" : "+v"(row), "+v"(col));
        }
    } else {
        int row = row0, col = col0;
        for (std::int64_t e = first; e < total; e += kStep) {
            const unsigned key = key_at(row, col);
            low = min(low, key);
            high = max(high, key);
            advance(row, col);
        }
    }
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1) {
        low = min(low, static_cast<unsigned>(__shfl_xor(static_cast<int>(low), offset)));
        high = max(high, static_cast<unsigned>(__shfl_xor(static_cast<int>(high), offset)));
    }
    if (lane == 0) {
        wave_low[wave] = low;
        wave_high[wave] = high;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        low = min(low, wave_low[w]);
        high = max(high, wave_high[w]);
    }
    const unsigned smallest = low;
    if constexpr (kKeys > 0) {
        const int r = in_range();
#pragma unroll
        for (int u = 0; u < kKeys; ++u) keys[u] = u * kWave < r ? keys[u] - smallest : 0u;
    }
    // visit(e, key) with key relative to the smallest, for every tile of
    // this thread (kKeys > 0: also those past the end, which a store leaves out).
    auto for_each_tile = [&](auto&& visit) {
        if constexpr (kKeys > 0) {
#pragma unroll
            for (int u = 0; u < kKeys; ++u) visit(static_cast<std::int64_t>(first + u * kWave), keys[u]);
        } else {
            int row = row0, col = col0;
            for (std::int64_t e = first; e < total; e += kStep) {
                visit(e, key_at(row, col) - smallest);
                advance(row, col);
            }
        }
    };
    // Passes from the top of the range down to bit 0: the first takes up to
    // kDigitBits bits (the keys are densest there, so the widest histogram
    // spreads them most), the others split the rest evenly.
    const unsigned range = high - smallest;
    const int bits = range ? 32 - __clz(static_cast<int>(range)) : 1;
    const int passes = (bits + kDigitBits - 1) / kDigitBits;
    const int first_width = min(bits, kDigitBits);
    const int width = passes > 1 ? (bits - first_width + passes - 2) / (passes - 1) : first_width;
    unsigned prefix = 0, mask = 0;
    int shift = bits;
    for (int pass = 0; pass < passes; ++pass) {
        const int next = max(shift - (pass == 0 ? first_width : width), 0);
        const unsigned digits = shift - next;
        for (int b = t; b < kBins; b += kSelectThreads) histogram[b] = 0;
        __syncthreads();
        for_each_tile([&](std::int64_t, unsigned key) {
            if ((key & mask) == prefix) atomicAdd(&histogram[__builtin_amdgcn_ubfe(key, next, digits)], 1u);
        });
        const unsigned need = still_needed;
        __syncthreads();
        // Thread t holds bins kBins - 1 - 2t and kBins - 2 - 2t (largest
        // first); a scan over threads counts the keys above each thread's
        // bins, and the thread whose bins reach the still-needed rank picks.
        const unsigned top = histogram[kBins - 1 - 2 * t], below_top = histogram[kBins - 2 - 2 * t];
        const unsigned sum = top + below_top;
        unsigned inclusive = sum;
#pragma unroll
        for (int offset = 1; offset < kWave; offset <<= 1) {
            const unsigned up = __shfl_up(inclusive, offset);
            if (lane >= offset) inclusive += up;
        }
        if (lane == kWave - 1) wave_low[wave] = inclusive;
        __syncthreads();
        unsigned above = inclusive - sum;
        for (int w = 0; w < wave; ++w) above += wave_low[w];
        if (above < need && above + sum >= need) {
            const bool in_top = above + top >= need;
            chosen_digit = static_cast<unsigned>(in_top ? kBins - 1 - 2 * t : kBins - 2 - 2 * t);
            still_needed = in_top ? need - above : need - above - top;
            equal_keys = in_top ? top : below_top;
        }
        __syncthreads();
        prefix |= chosen_digit << next;
        mask |= ((1u << digits) - 1u) << next;
        shift = next;
    }
    // prefix = the count-th largest key; still_needed = how many of the keys
    // equal to it are FP16 (the lowest indices), equal_keys how many there are.
    const unsigned ties = still_needed;
    if (ties == equal_keys) {
        if constexpr (kKeys > 0) {
            const int r = in_range();
#pragma unroll
            for (int u = 0; u < kKeys; ++u)
                if (u * kWave < r) out[first + u * kWave] = keys[u] >= prefix ? kFp16 : kInt8;
        } else {
            for_each_tile([&](std::int64_t e, unsigned key) { out[e] = key >= prefix ? kFp16 : kInt8; });
        }
        return;
    }
    auto lanes_below = [&](unsigned long long ballot) {
        return __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(ballot >> 32),
                                         __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(ballot), 0u));
    };
    if constexpr (kKeys > 0) {
        unsigned mine = 0;
#pragma unroll
        for (int u = 0; u < kKeys; ++u) mine += static_cast<unsigned>(__popcll(__ballot(keys[u] == prefix)));
        if (lane == 0) wave_low[wave] = mine;
        __syncthreads();
        unsigned before = 0;
        for (int w = 0; w < wave; ++w) before += wave_low[w];
        const int r = in_range();
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            const bool equal = keys[u] == prefix;
            const unsigned long long ballot = __ballot(equal);
            if (u * kWave < r)
                out[first + u * kWave] =
                    (keys[u] > prefix || (equal && before + lanes_below(ballot) < ties)) ? kFp16 : kInt8;
            before += static_cast<unsigned>(__popcll(ballot));
        }
    } else {
        // Chunk by chunk of 1024 tiles: ties before this one are those of
        // earlier chunks, earlier waves and earlier lanes.
        unsigned ties_before = 0;
        int row = row0, col = col0;
        for (std::int64_t base = 0; base < total; base += kSelectThreads) {
            const std::int64_t e = base + t;
            const unsigned key = e < total ? key_at(row, col) - smallest : 0u;
            const bool equal = e < total && key == prefix;
            const unsigned long long ballot = __ballot(equal);
            if (lane == 0) wave_low[wave] = static_cast<unsigned>(__popcll(ballot));
            __syncthreads();
            unsigned earlier = 0, all = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                earlier += w < wave ? wave_low[w] : 0u;
                all += wave_low[w];
            }
            if (e < total)
                out[e] = (key > prefix || (equal && ties_before + earlier + lanes_below(ballot) < ties)) ? kFp16
                                                                                                        : kInt8;
            ties_before += all;
            __syncthreads();
            advance(row, col);
        }
    }
}

// One wave per (head, coarse tile row i): bit b of word w is group 64w + b,
// whose key tiles lie in coarse tile (kt * 32) / tile_keys; lane b reads
// that code and two ballots form the route and skip words. Every 16-row
// query tile the coarse row covers gets the same words, so the wave computes
// them once and its lanes store the copies.
__global__ __launch_bounds__(256) void pack_kernel(const std::uint8_t* codes, int heads, int q_tiles16,
                                                   int words_per_row, int groups, int key_tiles_per_group,
                                                   int tiles_q, int tiles_k, int tile_rows, int tile_keys,
                                                   std::uint64_t* route_words, std::uint64_t* skip_words) {
    const std::int64_t wave = (static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (wave >= static_cast<std::int64_t>(heads) * tiles_q) return;  // whole waves
    const std::int64_t head = wave / tiles_q;
    const int i = static_cast<int>(wave % tiles_q);
    const std::uint8_t* row = codes + wave * tiles_k;
    const int qt0 = i * (tile_rows / kCellRows);
    const int copies = min(tile_rows / kCellRows, q_tiles16 - qt0);
    const std::int64_t out = (head * q_tiles16 + qt0) * words_per_row;
    for (int w = 0; w < words_per_row; ++w) {
        const int group = 64 * w + lane;
        std::uint8_t code = kFp16;
        if (group < groups) {
            const std::int64_t kt = static_cast<std::int64_t>(group) * key_tiles_per_group;
            code = row[kt * kCellKeys / tile_keys];
        }
        const std::uint64_t route = __ballot(code == kInt8);
        const std::uint64_t skip = __ballot(code == kSkip);
        for (int r = lane; r < copies; r += kWave) {
            route_words[out + static_cast<std::int64_t>(r) * words_per_row + w] = route;
            skip_words[out + static_cast<std::int64_t>(r) * words_per_row + w] = skip;
        }
    }
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
    const int tiles_q = (M - 1) / tile_rows + 1, tiles_k = (N - 1) / tile_keys + 1;
    const std::int64_t lanes = static_cast<std::int64_t>(heads) * tiles_q * kWave;
    if (!grid_ok(words, 256) || !grid_ok(lanes, 256)) return hipErrorInvalidConfiguration;
    pack_kernel<<<blocks_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
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
        // The first call on a device may come while the caller's stream is
        // being captured into a graph. The lookup enqueues no work, so this
        // thread's capture mode is relaxed around it (a global-mode capture
        // would otherwise reject the runtime call and invalidate the graph),
        // then restored.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        status = hipThreadExchangeStreamCaptureMode(&mode);
        if (status != hipSuccess) return status;
        void* ptr = nullptr;
        status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        const hipError_t restored = hipThreadExchangeStreamCaptureMode(&mode);
        if (status != hipSuccess) return status;
        if (restored != hipSuccess) return restored;
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
    const dim3 grid(static_cast<unsigned>(tiles_q + tiles_k), static_cast<unsigned>(heads));
    const bool vector = d % 8 == 0 && reinterpret_cast<std::uintptr_t>(Q) % 16 == 0 &&
                        reinterpret_cast<std::uintptr_t>(K) % 16 == 0 && (qs * 2) % 16 == 0 && (ks * 2) % 16 == 0;
    if (vector)
        tile_absmax_kernel<true><<<grid, 256, 0, s>>>(Q, K, M, N, d, qs, ks, tiles_q, tiles_k, tile_rows, tile_keys,
                                                      workspace);
    else
        tile_absmax_kernel<false><<<grid, 256, 0, s>>>(Q, K, M, N, d, qs, ks, tiles_q, tiles_k, tile_rows, tile_keys,
                                                       workspace);
    hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    const std::size_t lds = static_cast<std::size_t>(tiles_q + tiles_k) * sizeof(float);
    const unsigned blocks = static_cast<unsigned>(heads);
    if (total <= 8 * kSelectThreads)
        importance_select_kernel<8><<<blocks, kSelectThreads, lds, s>>>(workspace, tiles_q, tiles_k, count, tile_codes);
    else if (total <= 32 * kSelectThreads)
        importance_select_kernel<32><<<blocks, kSelectThreads, lds, s>>>(workspace, tiles_q, tiles_k, count,
                                                                          tile_codes);
    else
        importance_select_kernel<0><<<blocks, kSelectThreads, lds, s>>>(workspace, tiles_q, tiles_k, count, tile_codes);
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
