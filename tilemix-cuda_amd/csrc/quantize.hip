// Block INT8 quantizer for TileMix on gfx950.
//
// Replaces quantize_tilemix_qk / quantize_blocks<BlockRows> of the reference
// (src/tilemix.cu:16-49, 223-236). One 256-thread workgroup owns one
// quantization block (128 Q rows or 64 K rows x d features). Because rows are
// contiguous, a block is one contiguous span of rows*d halves: the vector path
// reads it once with 16-byte loads into registers (at most 8 per thread),
// reduces the absmax across the workgroup and quantizes from registers, so HBM
// sees exactly one read of the input and one write of the int8 output. The
// absmax runs on packed fp16 pairs (magnitudes by clearing the sign bits) and
// the per-element quotient uses the block's reciprocal with an exact
// correction step instead of a division (quantize_value_recip).

#include "tilemix_device.h"
#include "tilemix_launch.h"

#include <algorithm>

namespace tilemix {
namespace {

constexpr int kQuantThreads = 256;
constexpr int kQuantMaxChunks = (128 * 128 / 8) / kQuantThreads;  // 16-byte chunks per thread

// kContiguous: rows are d elements apart, so a block is one span of
// rows * d halves; otherwise chunk c of the block is chunk c % (d / 8) of row
// c / (d / 8). kChunks: 16-byte chunks held per thread, enough for the
// larger block of the launch (4 for 64 x 128 K blocks, 8 for 128 x 128 Q).
template <bool kVector, bool kContiguous, int kChunks = kQuantMaxChunks>
__global__ __launch_bounds__(kQuantThreads) void quantize_blocks_kernel(QuantSide q, QuantSide k, int d) {
    __shared__ float partial[kQuantThreads / kWave];
    __shared__ unsigned partial_bits[kQuantThreads / kWave];
    const bool is_q = static_cast<int>(blockIdx.x) < q.blocks;
    const QuantSide side = is_q ? q : k;
    const int block = is_q ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) - q.blocks;
    const std::int64_t head = blockIdx.y;
    const int first = block * side.block_rows;
    const int last = min(side.rows, first + side.block_rows);
    const int count = (last - first) * d;
    const std::uint16_t* in = side.x + head * side.in_head_stride + static_cast<std::int64_t>(first) * side.in_row_stride;
    const std::int64_t row_stride = side.in_row_stride;
    std::int8_t* out = side.x8 + head * static_cast<std::int64_t>(side.rows) * d +
                       static_cast<std::int64_t>(first) * d;
    const int t = threadIdx.x;

    uint4v chunk[kChunks];
    const int chunks = count / 8;
    float absmax = 0.0f;
    if constexpr (kVector) {
        // Chunks past the block's end load its last chunk again (in-block
        // values, which leave the maximum unchanged; they are not stored).
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int index = t + c * kQuantThreads;
            const int at = index < chunks ? index : chunks - 1;
            const std::uint16_t* source;
            if constexpr (kContiguous) {
                source = in + 8 * at;
            } else {
                const int per_row = d / 8;
                source = in + (at / per_row) * row_stride + 8 * (at % per_row);
            }
            chunk[c] = *reinterpret_cast<const uint4v*>(source);
        }
        // |x| as fp16 bit patterns: unsigned order is float order for them,
        // NaN patterns (> 0x7c00) sorting above +inf.
        unsigned top = 0;
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
#pragma unroll
            for (int w = 0; w < 4; ++w) top = max_u16x2(top, chunk[c][w] & 0x7fff7fffu);
        unsigned bits = wave_max_bits(max(top & 0xffffu, top >> 16));
        if ((t & (kWave - 1)) == 0) partial_bits[t / kWave] = bits;
        __syncthreads();
        bits = max(max(partial_bits[0], partial_bits[1]), max(partial_bits[2], partial_bits[3]));
        if (bits > 0x7c00u) {
            // A NaN in the block: the maximum skips NaNs, as fmaxf does.
            unsigned clean = 0;
#pragma unroll
            for (int c = 0; c < kChunks; ++c)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned h = (chunk[c][e / 2] >> (16 * (e % 2))) & 0x7fffu;
                    clean = h <= 0x7c00u ? max(clean, h) : clean;
                }
            clean = wave_max_bits(clean);
            __syncthreads();
            if ((t & (kWave - 1)) == 0) partial_bits[t / kWave] = clean;
            __syncthreads();
            bits = max(max(partial_bits[0], partial_bits[1]), max(partial_bits[2], partial_bits[3]));
        }
        absmax = half_bits_to_float(static_cast<std::uint16_t>(bits));
    } else {
        for (int index = t; index < count; index += kQuantThreads)
            absmax = fmaxf(absmax, fabsf(half_bits_to_float(in[(index / d) * row_stride + index % d])));
        absmax = wave_max(absmax);
        if ((t & (kWave - 1)) == 0) partial[t / kWave] = absmax;
        __syncthreads();
        absmax = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
    }
    const float scale = block_scale(absmax);
    const float recip = 1.0f / scale;  // used only when scale > 0
    if (t == 0) side.scales[head * side.blocks + block] = float_to_half_bits(scale);

    if constexpr (kVector) {
        if (scale > 0.0f) {
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int index = t + c * kQuantThreads;
                if (index < chunks) {
                    int v[8];
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        v[e] = quantize_half<0>(chunk[c][e / 2], scale, recip);
                        v[e + 1] = quantize_half<1>(chunk[c][e / 2], scale, recip);
                    }
                    uint2v packed;
                    packed[0] = pack_bytes(v[0], v[1], v[2], v[3]);
                    packed[1] = pack_bytes(v[4], v[5], v[6], v[7]);
                    reinterpret_cast<uint2v*>(out)[index] = packed;
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int index = t + c * kQuantThreads;
                if (index < chunks) reinterpret_cast<uint2v*>(out)[index] = uint2v{0u, 0u};
            }
        }
    } else {
        for (int index = t; index < count; index += kQuantThreads)
            out[index] = static_cast<std::int8_t>(
                quantize_value_recip(half_bits_to_float(in[(index / d) * row_stride + index % d]), scale, recip));
    }
}

bool aligned(const void* pointer, std::size_t bytes) {
    return (reinterpret_cast<std::uintptr_t>(pointer) % bytes) == 0;
}

}  // namespace

hipError_t launch_quantize(const QuantSide& q, const QuantSide& k, int heads, int d,
                           hipStream_t stream) {
    const int blocks = q.blocks + k.blocks;
    if (blocks == 0) return hipSuccess;
    if (heads > 65535) return hipErrorInvalidConfiguration;
    // The vector path reads 16-byte chunks of halves and writes 8-byte chunks
    // of int8; rows of d % 8 == 0 halves keep every block start aligned.
    bool vector = d % 8 == 0;
    bool contiguous = true;
    for (const QuantSide* side : {&q, &k}) {
        if (side->blocks == 0) continue;
        vector = vector && aligned(side->x, 16) && aligned(side->x8, 8) &&
                 (side->in_head_stride * 2) % 16 == 0 && (side->in_row_stride * 2) % 16 == 0;
        contiguous = contiguous && side->in_row_stride == d;
    }
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(heads));
    // Chunks of 16 bytes per thread the larger block of the launch needs.
    std::int64_t need = 0;
    for (const QuantSide* side : {&q, &k})
        if (side->blocks) need = std::max<std::int64_t>(need, static_cast<std::int64_t>(side->block_rows) * d / 8);
    const bool small = need <= 4 * kQuantThreads;
    if (vector && contiguous && small)
        quantize_blocks_kernel<true, true, 4><<<grid, kQuantThreads, 0, stream>>>(q, k, d);
    else if (vector && contiguous)
        quantize_blocks_kernel<true, true><<<grid, kQuantThreads, 0, stream>>>(q, k, d);
    else if (vector && small)
        quantize_blocks_kernel<true, false, 4><<<grid, kQuantThreads, 0, stream>>>(q, k, d);
    else if (vector)
        quantize_blocks_kernel<true, false><<<grid, kQuantThreads, 0, stream>>>(q, k, d);
    else
        quantize_blocks_kernel<false, false><<<grid, kQuantThreads, 0, stream>>>(q, k, d);
    return hipGetLastError();
}

QuantSide make_quant_side(const std::uint16_t* x, std::int8_t* x8, std::uint16_t* scales,
                          std::int64_t head_stride, int rows, int block_rows, std::int64_t row_stride) {
    QuantSide side{};
    side.x = x;
    side.x8 = x8;
    side.scales = scales;
    side.in_head_stride = head_stride;
    side.in_row_stride = row_stride;
    side.rows = rows;
    side.block_rows = block_rows;
    side.blocks = x ? (rows - 1) / block_rows + 1 : 0;
    return side;
}

}  // namespace tilemix

extern "C" int tilemix_quantize_qk(const std::uint16_t* Q, const std::uint16_t* K, std::int8_t* Q8,
                                   std::int8_t* K8, std::uint16_t* q_scales, std::uint16_t* k_scales,
                                   int M, int N, int d, void* stream) {
    // Validation order of src/tilemix.cu:227-230.
    if (!Q || !K || !Q8 || !K8 || !q_scales || !k_scales || M <= 0 || N <= 0 || d <= 0)
        return hipErrorInvalidValue;
    if (d > tilemix::kMaxHeadDim) return hipErrorNotSupported;
    const auto q = tilemix::make_quant_side(Q, Q8, q_scales, 0, M, tilemix::kQBlockRows, d);
    const auto k = tilemix::make_quant_side(K, K8, k_scales, 0, N, tilemix::kKBlockRows, d);
    return tilemix::launch_quantize(q, k, 1, d, static_cast<hipStream_t>(stream));
}

extern "C" int tilemix_quantize_qk_strided(const std::uint16_t* Q, const std::uint16_t* K,
                                           std::int8_t* Q8, std::int8_t* K8,
                                           std::uint16_t* q_scales, std::uint16_t* k_scales,
                                           int heads, int M, int N, int d,
                                           std::int64_t q_head_stride, std::int64_t k_head_stride,
                                           std::int64_t q_row_stride, std::int64_t k_row_stride,
                                           void* stream) {
    const bool q_side = Q || Q8 || q_scales;
    const bool k_side = K || K8 || k_scales;
    if ((q_side && (!Q || !Q8 || !q_scales)) || (k_side && (!K || !K8 || !k_scales)) ||
        (!q_side && !k_side) || heads <= 0 || d <= 0 || (q_side && M <= 0) || (k_side && N <= 0))
        return hipErrorInvalidValue;
    const std::int64_t q_row = q_row_stride ? q_row_stride : d;
    const std::int64_t k_row = k_row_stride ? k_row_stride : d;
    if ((q_side && !tilemix::strided_heads_ok(heads, M, d, q_head_stride, q_row)) ||
        (k_side && !tilemix::strided_heads_ok(heads, N, d, k_head_stride, k_row)))
        return hipErrorInvalidValue;
    if (d > tilemix::kMaxHeadDim) return hipErrorNotSupported;
    const auto q = tilemix::make_quant_side(q_side ? Q : nullptr, Q8, q_scales, q_head_stride,
                                            q_side ? M : 1, tilemix::kQBlockRows, q_row);
    const auto k = tilemix::make_quant_side(k_side ? K : nullptr, K8, k_scales, k_head_stride,
                                            k_side ? N : 1, tilemix::kKBlockRows, k_row);
    return tilemix::launch_quantize(q, k, heads, d, static_cast<hipStream_t>(stream));
}

extern "C" int tilemix_quantize_qk_batched(const std::uint16_t* Q, const std::uint16_t* K,
                                           std::int8_t* Q8, std::int8_t* K8,
                                           std::uint16_t* q_scales, std::uint16_t* k_scales,
                                           int heads, int M, int N, int d,
                                           std::int64_t q_head_stride, std::int64_t k_head_stride,
                                           void* stream) {
    return tilemix_quantize_qk_strided(Q, K, Q8, K8, q_scales, k_scales, heads, M, N, d, q_head_stride,
                                       k_head_stride, 0, 0, stream);
}
