// Routed INT8/FP16 fused attention for gfx950 (MI355X).
//
// Replaces fused_fp16_attention + launch_fused_fp16_attention of the reference
// (src/tilemix.cu:51-220, 238-278). Design (not a translation):
//
//  * A 256-thread workgroup (4 wave64s) owns 128 query rows of one head - one
//    Q quantization block - and streams the keys in 64-key tiles, one K
//    quantization block each, so q_scale is constant per workgroup and
//    k_scale per tile.
//  * Each wave owns 32 query rows (two 16-row routing cells tall). Scores are
//    computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16 (FP16
//    cells) or v_mfma_i32_16x16x64_i8 (INT8 cells, exact int32 dots). In that
//    layout lane (g, i) holds four consecutive keys of query row i, so the
//    online-softmax state of a row lives in lanes i, i+16, i+32, i+48 and
//    needs only two cross-lane steps.
//  * The probabilities stay in registers and feed O^T += V^T P^T on
//    v_mfma_f32_16x16x32_f16; the V^T operand is read from the row-major V
//    tile in LDS with ds_read_b64_tr_b16, which transposes 16-bit elements
//    across each 16-lane group. Key order inside a 32-key MFMA step is
//    permuted identically on both operands.
//  * A 16x32 routing cell covers whole 16x16 MFMA blocks, so each route is
//    uniform per MFMA and the branch is taken on scalar route bits.
//  * The optional in-kernel Q quantization reproduces quantize_tilemix_qk's
//    bytes exactly: the workgroup's 128 rows are exactly one Q block.

#include "tilemix_device.h"
#include "tilemix_launch.h"
#include "tilemix_capi.h"

#include <atomic>
#include <cmath>
#include <cstring>

namespace tilemix {
namespace {

constexpr int kThreadsPerGroup = 256;
constexpr int kRowsPerGroup = 128;  // one Q quantization block
constexpr int kRowsPerWave = 32;
constexpr int kTileKeys = 64;  // one K quantization block
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const std::uint16_t* Q;
    const std::uint16_t* K;
    const std::uint16_t* V;
    float* O;
    const std::int8_t* Q8;
    const std::int8_t* K8;
    const std::uint16_t* q_scales;
    const std::uint16_t* k_scales;
    const std::uint64_t* route_words;
    const std::uint64_t* skip_words;
    std::uint8_t* trace;
    std::int32_t* dots;
    std::int8_t* q8_out;
    std::uint16_t* q_scales_out;
    std::int64_t q_stride;
    std::int64_t k_stride;
    std::int64_t v_stride;
    std::int64_t o_stride;
    std::int64_t words_per_row;
    std::int64_t words_per_head;
    int heads;
    int M;
    int N;
    int d;
    int key_tiles_per_group;
    int q_tiles16;
    int key_tiles32;
    int q_blocks;
    int k_blocks;
    int causal;
    int fuse_q_quant;
    int int8_operands;
    float score_log2;  // score_scale * log2(e)
    float score_scale;
};

// Route code of one 16x32 cell: 0 = FP16, 1 = INT8, 2 = skip. Cells outside
// the problem report skip so that no work is done for them.
__device__ __forceinline__ int cell_code(const AttnParams& p, std::int64_t head, int qt, int kt) {
    if (qt >= p.q_tiles16 || kt >= p.key_tiles32) return 2;
    const std::int64_t group = kt / p.key_tiles_per_group;
    const std::int64_t word = head * p.words_per_head + qt * p.words_per_row + (group >> 6);
    const unsigned bit = static_cast<unsigned>(group & 63);
    if (p.skip_words && ((p.skip_words[word] >> bit) & 1u)) return 2;
    if (p.route_words && ((p.route_words[word] >> bit) & 1u)) return 1;
    return 0;
}

template <int DC>
struct Layout {
    static constexpr int kDP = 32 * DC;            // padded head dim, fp16 path
    static constexpr int kD8C = (DC + 1) / 2;      // 64-feature chunks, int8 path
    static constexpr int kDP8 = 64 * kD8C;
    static constexpr int kFB = kDP / 16;           // 16-feature output blocks
    static constexpr int kKStride = kDP * 2 + 16;  // bytes per K row in LDS
    static constexpr int kVStride = kDP * 2 + 32;  // bytes per V row in LDS
    static constexpr int kK8Stride = kDP8 + 16;    // bytes per K8 row in LDS
    static constexpr int kKBytes = kTileKeys * kKStride;
    static constexpr int kVBytes = kTileKeys * kVStride;
    static constexpr int kK8Bytes = kTileKeys * kK8Stride;
    static constexpr int kQ8Stride = kDP8 + 16;    // prologue staging of quantized Q
    static constexpr int kSmemBytes = kKBytes + kVBytes + kK8Bytes;
    static_assert(kRowsPerGroup * kQ8Stride <= kSmemBytes, "Q8 staging must fit the tile area");
};

__device__ __forceinline__ half8 concat(half4 a, half4 b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ half4 read_tr16(const unsigned char* lds_byte_address) {
    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lds_byte_address));
    return __builtin_bit_cast(half4, raw);
}

template <int DC, bool kVector, bool kPrecise>
__global__ __launch_bounds__(kThreadsPerGroup, 2) void attention_kernel(const AttnParams p) {
    using L = Layout<DC>;
    constexpr int kDP = L::kDP;
    constexpr int kD8C = L::kD8C;
    constexpr int kFB = L::kFB;
    __shared__ __attribute__((aligned(16))) unsigned char smem[L::kSmemBytes];
    __shared__ float group_max[kThreadsPerGroup / kWave];
    unsigned char* const lds_k = smem;
    unsigned char* const lds_v = smem + L::kKBytes;
    unsigned char* const lds_k8 = smem + L::kKBytes + L::kVBytes;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int i = lane & 15;

    // Heaviest causal tiles first: block index -> (q block, head).
    const int linear = blockIdx.x;
    const int qblock = p.causal ? p.q_blocks - 1 - linear / p.heads : linear / p.heads;
    const std::int64_t head = linear % p.heads;
    const int q0 = qblock * kRowsPerGroup;
    const int qw = q0 + wave * kRowsPerWave;
    const int M = p.M, N = p.N, d = p.d;

    const std::uint16_t* Qh = p.Q + head * p.q_stride;
    const std::uint16_t* Kh = p.K + head * p.k_stride;
    const std::uint16_t* Vh = p.V + head * p.v_stride;
    float* Oh = p.O + head * p.o_stride;

    // ---------------------------------------------------------------- Q
    half8 qf[2][DC];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = qw + 16 * b + i;
#pragma unroll
        for (int dc = 0; dc < DC; ++dc) {
            const int feature = 32 * dc + 8 * g;
            if constexpr (kVector) {
                qf[b][dc] = (row < M && feature < d)
                    ? *reinterpret_cast<const half8*>(Qh + static_cast<std::int64_t>(row) * d + feature)
                    : half8{};
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qf[b][dc][e] = (row < M && feature + e < d)
                        ? __builtin_bit_cast(_Float16, Qh[static_cast<std::int64_t>(row) * d + feature + e])
                        : static_cast<_Float16>(0.0f);
            }
        }
    }

    int4v q8f[2][kD8C];
    float q_scale = 0.0f;
    if (p.int8_operands) {
        if (p.fuse_q_quant) {
            // The workgroup's rows are exactly one 128-row Q block.
            float absmax = 0.0f;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int dc = 0; dc < DC; ++dc)
#pragma unroll
                    for (int e = 0; e < 8; ++e) absmax = fmaxf(absmax, fabsf(static_cast<float>(qf[b][dc][e])));
            absmax = wave_max(absmax);
            if (lane == 0) group_max[wave] = absmax;
            __syncthreads();
            absmax = fmaxf(fmaxf(group_max[0], group_max[1]), fmaxf(group_max[2], group_max[3]));
            const float scale = block_scale(absmax);
            const _Float16 stored = static_cast<_Float16>(scale);
            q_scale = static_cast<float>(stored);
            if (tid == 0 && p.q_scales_out)
                p.q_scales_out[head * p.q_blocks + qblock] = __builtin_bit_cast(std::uint16_t, stored);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int local = wave * kRowsPerWave + 16 * b + i;
                const int row = q0 + local;
#pragma unroll
                for (int dc = 0; dc < 2 * kD8C; ++dc) {
                    int v[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        v[e] = dc < DC ? quantize_value(static_cast<float>(qf[b][dc < DC ? dc : 0][e]), scale) : 0;
                    uint2v packed;
                    packed[0] = pack_bytes(v[0], v[1], v[2], v[3]);
                    packed[1] = pack_bytes(v[4], v[5], v[6], v[7]);
                    const int feature = 32 * dc + 8 * g;
                    *reinterpret_cast<uint2v*>(smem + local * L::kQ8Stride + feature) = packed;
                    if (p.q8_out && row < M && feature < d) {
                        std::int8_t* dst = p.q8_out + head * static_cast<std::int64_t>(M) * d +
                                           static_cast<std::int64_t>(row) * d + feature;
                        if constexpr (kVector) {
                            *reinterpret_cast<uint2v*>(dst) = packed;
                        } else {
                            for (int e = 0; e < 8 && feature + e < d; ++e) dst[e] = static_cast<std::int8_t>(v[e]);
                        }
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int local = wave * kRowsPerWave + 16 * b + i;
#pragma unroll
                for (int m = 0; m < kD8C; ++m)
                    q8f[b][m] = *reinterpret_cast<const int4v*>(smem + local * L::kQ8Stride + 64 * m + 16 * g);
            }
            __syncthreads();  // staging area is reused by the key tiles
        } else {
            q_scale = half_bits_to_float(p.q_scales[head * p.q_blocks + qblock]);
            const std::int8_t* Q8h = p.Q8 + head * static_cast<std::int64_t>(M) * d;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int row = qw + 16 * b + i;
#pragma unroll
                for (int m = 0; m < kD8C; ++m) {
                    const int feature = 64 * m + 16 * g;
                    if constexpr (kVector) {
                        q8f[b][m] = (row < M && feature < d)
                            ? *reinterpret_cast<const int4v*>(Q8h + static_cast<std::int64_t>(row) * d + feature)
                            : int4v{0, 0, 0, 0};
                    } else {
                        unsigned char bytes[16];
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            bytes[e] = (row < M && feature + e < d)
                                ? static_cast<unsigned char>(Q8h[static_cast<std::int64_t>(row) * d + feature + e])
                                : 0;
                        q8f[b][m] = __builtin_bit_cast(int4v, bytes);
                    }
                }
            }
        }
    }

    // ---------------------------------------------------------- key loop
    float4v o[2][kFB];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int fb = 0; fb < kFB; ++fb) o[b][fb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};

    const int key_tiles64 = (N - 1) / kTileKeys + 1;
    int tiles = key_tiles64;
    if (p.causal) tiles = min(tiles, (q0 + kRowsPerGroup - 1) / kTileKeys + 1);
    const int qt0 = q0 / 16;
    const std::int64_t trace_base = head * static_cast<std::int64_t>(p.q_tiles16) * p.key_tiles32;

    for (int j = 0; j < tiles; ++j) {
        const int k0 = j * kTileKeys;
        // Route codes of the workgroup's 8 x 2 cells: lane c < 16 decodes cell
        // (row c / 2, key half c % 2); the ballots make the masks wave-uniform.
        int code = 2;
        if (lane < 16) code = cell_code(p, head, qt0 + (lane >> 1), 2 * j + (lane & 1));
        const std::uint32_t int8_mask = static_cast<std::uint32_t>(__ballot(lane < 16 && code == 1));
        const std::uint32_t skip_mask = static_cast<std::uint32_t>(__ballot(lane < 16 && code == 2));
        if (p.trace && wave == 0 && lane < 16) {
            const int qt = qt0 + (lane >> 1), kt = 2 * j + (lane & 1);
            if (qt < p.q_tiles16 && kt < p.key_tiles32)
                p.trace[trace_base + static_cast<std::int64_t>(qt) * p.key_tiles32 + kt] =
                    static_cast<std::uint8_t>(code);
        }
        if (skip_mask == 0xffffu) continue;  // whole 128x64 tile skipped (uniform across the group)
        const bool need16 = ((~int8_mask & ~skip_mask) & 0xffffu) != 0;
        const bool need8 = int8_mask != 0;

        // ---- cooperative tile loads into LDS
        if constexpr (kVector) {
            constexpr int kChunks16 = kDP / 8;  // 16-byte chunks per fp16 row
#pragma unroll
            for (int it = 0; it < DC; ++it) {
                const int c = tid + it * kThreadsPerGroup;
                const int row = c / kChunks16, col = c % kChunks16;
                const int key = k0 + row;
                const bool valid = key < N && col * 8 < d;
                const std::int64_t offset = static_cast<std::int64_t>(key) * d + col * 8;
                const uint4v zero{0u, 0u, 0u, 0u};
                if (need16)
                    *reinterpret_cast<uint4v*>(lds_k + row * L::kKStride + col * 16) =
                        valid ? *reinterpret_cast<const uint4v*>(Kh + offset) : zero;
                *reinterpret_cast<uint4v*>(lds_v + row * L::kVStride + col * 16) =
                    valid ? *reinterpret_cast<const uint4v*>(Vh + offset) : zero;
            }
            if (need8) {
                const std::int8_t* K8h = p.K8 + head * static_cast<std::int64_t>(N) * d;
                constexpr int kChunks8 = L::kDP8 / 16;
#pragma unroll
                for (int it = 0; it < kD8C; ++it) {
                    const int c = tid + it * kThreadsPerGroup;
                    const int row = c / kChunks8, col = c % kChunks8;
                    const int key = k0 + row;
                    const bool valid = key < N && col * 16 < d;
                    *reinterpret_cast<uint4v*>(lds_k8 + row * L::kK8Stride + col * 16) =
                        valid ? *reinterpret_cast<const uint4v*>(K8h + static_cast<std::int64_t>(key) * d + col * 16)
                              : uint4v{0u, 0u, 0u, 0u};
                }
            }
        } else {
            for (int e = tid; e < kTileKeys * kDP; e += kThreadsPerGroup) {
                const int row = e / kDP, f = e % kDP;
                const int key = k0 + row;
                const bool valid = key < N && f < d;
                const std::int64_t offset = static_cast<std::int64_t>(key) * d + f;
                if (need16)
                    *reinterpret_cast<std::uint16_t*>(lds_k + row * L::kKStride + 2 * f) = valid ? Kh[offset] : 0;
                *reinterpret_cast<std::uint16_t*>(lds_v + row * L::kVStride + 2 * f) = valid ? Vh[offset] : 0;
            }
            if (need8) {
                const std::int8_t* K8h = p.K8 + head * static_cast<std::int64_t>(N) * d;
                for (int e = tid; e < kTileKeys * L::kDP8; e += kThreadsPerGroup) {
                    const int row = e / L::kDP8, f = e % L::kDP8;
                    const int key = k0 + row;
                    lds_k8[row * L::kK8Stride + f] =
                        (key < N && f < d) ? static_cast<unsigned char>(K8h[static_cast<std::int64_t>(key) * d + f]) : 0;
                }
            }
        }
        __syncthreads();

        const unsigned wave_int8 = (int8_mask >> (4 * wave)) & 0xfu;
        const unsigned wave_skip = (skip_mask >> (4 * wave)) & 0xfu;
        const bool wave_active = qw < M && wave_skip != 0xfu && !(p.causal && k0 > qw + kRowsPerWave - 1);
        if (wave_active) {
            float k_factor = 0.0f;  // q_scale * k_scale * score_scale * log2(e)
            if (wave_int8) {
                const float k_scale = half_bits_to_float(p.k_scales[head * p.k_blocks + j]);
                k_factor = ((q_scale * k_scale) * p.score_scale) * kLog2e;
            }
            const float f_factor = p.score_log2;

            // ---- scores S^T[kb][b]: lane (g, i) holds query i, keys 16kb + 4g + r
            float4v s[2][4];
            const bool uniform16 = wave_int8 == 0 && wave_skip == 0;
            if (uniform16) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    float4v acc0{0.0f, 0.0f, 0.0f, 0.0f}, acc1{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int dc = 0; dc < DC; ++dc) {
                        const half8 kf = *reinterpret_cast<const half8*>(
                            lds_k + (16 * kb + i) * L::kKStride + (32 * dc + 8 * g) * 2);
                        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[0][dc], acc0, 0, 0, 0);
                        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[1][dc], acc1, 0, 0, 0);
                    }
                    s[0][kb] = acc0 * f_factor;
                    s[1][kb] = acc1 * f_factor;
                }
            } else {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const int t = kb >> 1;
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const unsigned cell = 2 * b + t;
                        const bool skip = (wave_skip >> cell) & 1u;
                        const bool int8 = (wave_int8 >> cell) & 1u;
                        if (skip) {
                            s[b][kb] = float4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
                        } else if (int8) {
                            int4v acc{0, 0, 0, 0};
#pragma unroll
                            for (int m = 0; m < kD8C; ++m) {
                                const int4v kf = *reinterpret_cast<const int4v*>(
                                    lds_k8 + (16 * kb + i) * L::kK8Stride + 64 * m + 16 * g);
                                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, q8f[b][m], acc, 0, 0, 0);
                            }
                            if (p.dots) {
                                const int query = qw + 16 * b + i;
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    const int key = k0 + 16 * kb + 4 * g + r;
                                    if (query < M && key < N && !(p.causal && key > query))
                                        p.dots[head * static_cast<std::int64_t>(M) * N +
                                               static_cast<std::int64_t>(query) * N + key] = acc[r];
                                }
                            }
#pragma unroll
                            for (int r = 0; r < 4; ++r) s[b][kb][r] = static_cast<float>(acc[r]) * k_factor;
                        } else {
                            float4v acc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                            for (int dc = 0; dc < DC; ++dc) {
                                const half8 kf = *reinterpret_cast<const half8*>(
                                    lds_k + (16 * kb + i) * L::kKStride + (32 * dc + 8 * g) * 2);
                                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[b][dc], acc, 0, 0, 0);
                            }
                            s[b][kb] = acc * f_factor;
                        }
                    }
                }
            }

            // ---- element masks: key tail and causal diagonal
            if (k0 + kTileKeys > N || (p.causal && k0 + kTileKeys - 1 > qw)) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int query = qw + 16 * b + i;
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int key = k0 + 16 * kb + 4 * g + r;
                            if (key >= N || (p.causal && key > query)) s[b][kb][r] = -INFINITY;
                        }
                }
            }

            // ---- online softmax (log2 domain) and P.V
            half8 ph[2][2];
            half8 pl[2][2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                float tile_max = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) tile_max = fmaxf(tile_max, s[b][kb][r]);
                tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
                tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
                const float m_new = fmaxf(m_run[b], tile_max);
                const float m_use = m_new == -INFINITY ? 0.0f : m_new;
                const float alpha = __builtin_amdgcn_exp2f(m_run[b] - m_use);
                m_run[b] = m_new;
                float sum = 0.0f;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float pr = __builtin_amdgcn_exp2f(s[b][kb][r] - m_use);
                        s[b][kb][r] = pr;
                        sum += pr;
                    }
                l_run[b] = l_run[b] * alpha + sum;
#pragma unroll
                for (int fb = 0; fb < kFB; ++fb) o[b][fb] *= alpha;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float a = s[b][2 * ks][r], c = s[b][2 * ks + 1][r];
                        const _Float16 ha = static_cast<_Float16>(a), hc = static_cast<_Float16>(c);
                        ph[b][ks][r] = ha;
                        ph[b][ks][4 + r] = hc;
                        if constexpr (kPrecise) {
                            pl[b][ks][r] = static_cast<_Float16>(a - static_cast<float>(ha));
                            pl[b][ks][4 + r] = static_cast<_Float16>(c - static_cast<float>(hc));
                        }
                    }
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const unsigned char* v_lo = lds_v + (32 * ks + 4 * g + (i >> 2)) * L::kVStride + 8 * (i & 3);
                const unsigned char* v_hi = v_lo + 16 * L::kVStride;
#pragma unroll
                for (int fb = 0; fb < kFB; ++fb) {
                    const half8 vf = concat(read_tr16(v_lo + 32 * fb), read_tr16(v_hi + 32 * fb));
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        o[b][fb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[b][ks], o[b][fb], 0, 0, 0);
                        if constexpr (kPrecise)
                            o[b][fb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[b][ks], o[b][fb], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }

    // Routing trace of tiles a causal workgroup never visits.
    if (p.trace && wave == 0 && lane < 16) {
        for (int j = tiles; j < key_tiles64; ++j) {
            const int qt = qt0 + (lane >> 1), kt = 2 * j + (lane & 1);
            if (qt < p.q_tiles16 && kt < p.key_tiles32)
                p.trace[trace_base + static_cast<std::int64_t>(qt) * p.key_tiles32 + kt] =
                    static_cast<std::uint8_t>(cell_code(p, head, qt, kt));
        }
    }

    // ---------------------------------------------------------- epilogue
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float l = l_run[b];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const float inverse = l > 0.0f ? 1.0f / l : 0.0f;
        const int row = qw + 16 * b + i;
        if (row >= M) continue;
        float* out_row = Oh + static_cast<std::int64_t>(row) * d;
#pragma unroll
        for (int fb = 0; fb < kFB; ++fb) {
            const int feature = 16 * fb + 4 * g;
            const float4v value = o[b][fb] * inverse;
            if constexpr (kVector) {
                if (feature < d) *reinterpret_cast<float4v*>(out_row + feature) = value;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (feature + r < d) out_row[feature + r] = value[r];
            }
        }
    }
}

template <int DC, bool kVector, bool kPrecise>
hipError_t launch_variant(const AttnParams& p, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(p.q_blocks) * static_cast<unsigned>(p.heads);
    attention_kernel<DC, kVector, kPrecise><<<blocks, kThreadsPerGroup, 0, stream>>>(p);
    return hipGetLastError();
}

template <int DC>
hipError_t launch_dc(const AttnParams& p, bool vector, bool precise, hipStream_t stream) {
    if (vector)
        return precise ? launch_variant<DC, true, true>(p, stream) : launch_variant<DC, true, false>(p, stream);
    return precise ? launch_variant<DC, false, true>(p, stream) : launch_variant<DC, false, false>(p, stream);
}

bool aligned(const void* pointer, std::size_t bytes) {
    return (reinterpret_cast<std::uintptr_t>(pointer) % bytes) == 0;
}

std::size_t words_per_row(int N, int group) {
    const std::size_t key_tiles = (static_cast<std::size_t>(N) - 1) / kCellKeys + 1;
    const std::size_t groups = (key_tiles - 1) / static_cast<std::size_t>(group) + 1;
    return (groups - 1) / 64 + 1;
}

std::size_t word_count(int M, int N, int group) {
    if (M <= 0 || N <= 0 || group <= 0) return 0;
    return ((static_cast<std::size_t>(M) - 1) / kCellRows + 1) * words_per_row(N, group);
}

// gfx950 check, cached per device (the reference queries device properties
// on every call, src/tilemix.cu:254-260).
hipError_t check_device() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> verdict[kMaxDevices];  // 0 unknown, 1 supported, 2 unsupported
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return status;
    if (device >= 0 && device < kMaxDevices) {
        const int known = verdict[device].load(std::memory_order_relaxed);
        if (known == 1) return hipSuccess;
        if (known == 2) return hipErrorNotSupported;
    }
    hipDeviceProp_t properties{};
    status = hipGetDeviceProperties(&properties, device);
    if (status != hipSuccess) return status;
    const bool supported = std::strncmp(properties.gcnArchName, "gfx950", 6) == 0;
    if (device >= 0 && device < kMaxDevices) verdict[device].store(supported ? 1 : 2, std::memory_order_relaxed);
    return supported ? hipSuccess : hipErrorNotSupported;
}

hipError_t launch_attention(const AttnParams& p, bool precise, hipStream_t stream) {
    if (static_cast<long long>(p.q_blocks) * p.heads > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipError_t status = check_device();
    if (status != hipSuccess) return status;
    bool vector = p.d % 16 == 0 && aligned(p.Q, 16) && aligned(p.K, 16) && aligned(p.V, 16) &&
                  aligned(p.O, 16) && p.q_stride % 8 == 0 && p.k_stride % 8 == 0 &&
                  p.v_stride % 8 == 0 && p.o_stride % 4 == 0;
    if (p.int8_operands) {
        if (!p.fuse_q_quant) vector = vector && aligned(p.Q8, 16);
        if (p.q8_out) vector = vector && aligned(p.q8_out, 8);
        vector = vector && aligned(p.K8, 16);
    }
    const int dc = (p.d + 31) / 32;
    switch (dc) {
        case 1: return launch_dc<1>(p, vector, precise, stream);
        case 2: return launch_dc<2>(p, vector, precise, stream);
        case 3: return launch_dc<3>(p, vector, precise, stream);
        default: return launch_dc<4>(p, vector, precise, stream);
    }
}

AttnParams base_params(const std::uint16_t* Q, const std::uint16_t* K, const std::uint16_t* V, float* O,
                       int heads, int M, int N, int d, float score_scale, int group) {
    AttnParams p{};
    p.Q = Q;
    p.K = K;
    p.V = V;
    p.O = O;
    p.heads = heads;
    p.M = M;
    p.N = N;
    p.d = d;
    p.key_tiles_per_group = group;
    p.q_tiles16 = (M - 1) / kCellRows + 1;
    p.key_tiles32 = (N - 1) / kCellKeys + 1;
    p.q_blocks = (M - 1) / kQBlockRows + 1;
    p.k_blocks = (N - 1) / kKBlockRows + 1;
    p.words_per_row = static_cast<std::int64_t>(words_per_row(N, group));
    p.words_per_head = static_cast<std::int64_t>(word_count(M, N, group));
    p.score_scale = score_scale;
    p.score_log2 = score_scale * kLog2e;
    p.q_stride = static_cast<std::int64_t>(M) * d;
    p.k_stride = static_cast<std::int64_t>(N) * d;
    p.v_stride = static_cast<std::int64_t>(N) * d;
    p.o_stride = static_cast<std::int64_t>(M) * d;
    return p;
}

}  // namespace
}  // namespace tilemix

extern "C" int tilemix_attention(const std::uint16_t* Q, const std::uint16_t* K, const std::uint16_t* V,
                                 float* O, int M, int N, int d, float score_scale, void* stream,
                                 const std::uint64_t* route_words, std::size_t route_word_count,
                                 int key_tiles_per_group, std::uint8_t* decoded_bits,
                                 const std::int8_t* Q8, const std::int8_t* K8,
                                 const std::uint16_t* q_scales, const std::uint16_t* k_scales,
                                 std::int32_t* score_dots) {
    using namespace tilemix;
    // Validation order and codes of src/tilemix.cu:242-253; every argument
    // error returns before the first HIP runtime call.
    if (!Q || !K || !V || !O || M <= 0 || N <= 0 || d <= 0 || !std::isfinite(score_scale) ||
        key_tiles_per_group <= 0 || (!route_words && route_word_count != 0))
        return hipErrorInvalidValue;
    if (d > kMaxHeadDim) return hipErrorNotSupported;
    if (route_words && route_word_count < word_count(M, N, key_tiles_per_group)) return hipErrorInvalidValue;
    const bool has_quantized = Q8 && K8 && q_scales && k_scales;
    const bool any_quantized = Q8 || K8 || q_scales || k_scales || score_dots;
    if ((any_quantized && !has_quantized) || (route_words && !has_quantized)) return hipErrorInvalidValue;

    AttnParams p = base_params(Q, K, V, O, 1, M, N, d, score_scale, key_tiles_per_group);
    p.route_words = route_words;
    p.trace = decoded_bits;
    p.dots = route_words ? score_dots : nullptr;  // only INT8 cells write dots
    p.int8_operands = route_words != nullptr;
    p.Q8 = Q8;
    p.K8 = K8;
    p.q_scales = q_scales;
    p.k_scales = k_scales;
    // The per-head API keeps the reference's fp32-level accuracy (its own test
    // suite checks 1e-5 + 1e-4|x| against fp64), so P.V runs in split precision.
    return launch_attention(p, /*precise=*/true, static_cast<hipStream_t>(stream));
}

extern "C" int tilemix_attention_batched(const TileMixBatchedArgs* args, void* stream) {
    using namespace tilemix;
    if (!args) return hipErrorInvalidValue;
    const TileMixBatchedArgs& a = *args;
    const int group = a.key_tiles_per_group;
    if (!a.Q || !a.K || !a.V || !a.O || a.heads <= 0 || a.M <= 0 || a.N <= 0 || a.d <= 0 ||
        !std::isfinite(a.score_scale) || group <= 0)
        return hipErrorInvalidValue;
    if (a.d > kMaxHeadDim) return hipErrorNotSupported;
    if (a.heads > 1) {
        const std::int64_t qn = static_cast<std::int64_t>(a.M) * a.d;
        const std::int64_t kn = static_cast<std::int64_t>(a.N) * a.d;
        if (a.q_head_stride < qn || a.o_head_stride < qn || a.k_head_stride < kn || a.v_head_stride < kn)
            return hipErrorInvalidValue;
    }
    const bool int8 = a.route_words != nullptr;
    if (a.quantize < 0 || a.quantize > 2) return hipErrorInvalidValue;
    if (int8) {
        if (!a.K8 || !a.k_scales) return hipErrorInvalidValue;
        if (!a.quantize && (!a.Q8 || !a.q_scales)) return hipErrorInvalidValue;
        if (a.quantize && (!a.Q8) != (!a.q_scales)) return hipErrorInvalidValue;
    } else if (a.score_dots) {
        return hipErrorInvalidValue;
    }
    if (a.quantize == 1 && int8) {
        const QuantSide none = make_quant_side(nullptr, nullptr, nullptr, 0, 1, kQBlockRows);
        const QuantSide k = make_quant_side(a.K, a.K8, a.k_scales, a.k_head_stride, a.N, kKBlockRows);
        const hipError_t status = check_device();
        if (status != hipSuccess) return status;
        const hipError_t quant = launch_quantize(none, k, a.heads, a.d, static_cast<hipStream_t>(stream));
        if (quant != hipSuccess) return quant;
    }
    AttnParams p = base_params(a.Q, a.K, a.V, a.O, a.heads, a.M, a.N, a.d, a.score_scale, group);
    p.q_stride = a.q_head_stride;
    p.k_stride = a.k_head_stride;
    p.v_stride = a.v_head_stride;
    p.o_stride = a.o_head_stride;
    if (a.heads == 1) {
        p.q_stride = static_cast<std::int64_t>(a.M) * a.d;
        p.o_stride = p.q_stride;
        p.k_stride = static_cast<std::int64_t>(a.N) * a.d;
        p.v_stride = p.k_stride;
    }
    p.causal = a.causal != 0;
    p.route_words = a.route_words;
    p.skip_words = a.skip_words;
    p.trace = a.decoded_bits;
    p.dots = a.score_dots;
    p.int8_operands = int8;
    p.fuse_q_quant = int8 && a.quantize;
    p.Q8 = a.Q8;
    p.K8 = a.K8;
    p.q_scales = a.q_scales;
    p.k_scales = a.k_scales;
    if (p.fuse_q_quant) {
        p.q8_out = a.Q8;
        p.q_scales_out = a.q_scales;
    }
    return launch_attention(p, a.precise != 0, static_cast<hipStream_t>(stream));
}

extern "C" std::size_t tilemix_routing_words_per_row_c(int N, int key_tiles_per_group) {
    if (N <= 0 || key_tiles_per_group <= 0) return 0;
    return tilemix::words_per_row(N, key_tiles_per_group);
}

extern "C" std::size_t tilemix_routing_word_count_c(int M, int N, int key_tiles_per_group) {
    return tilemix::word_count(M, N, key_tiles_per_group);
}

extern "C" std::size_t tilemix_shared_bytes_c(int d, int quantized) {
    if (d <= 0 || d > tilemix::kMaxHeadDim) return 0;
    const std::size_t padded = static_cast<std::size_t>((d + 15) / 16) * 16;
    return 2 * padded * (16 + 2 * 32) + 4 * 16 * 32 + (quantized ? (16 + 32) * padded : 0);
}

extern "C" const char* tilemix_version(void) { return "tilemix-hip 0.1 gfx950"; }
