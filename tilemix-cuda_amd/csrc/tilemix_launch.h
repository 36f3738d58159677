#pragma once
// Host-side declarations shared by the TileMix translation units.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace tilemix {

inline constexpr int kMaxHeadDim = 128;  // kFusedMaxHeadDim
inline constexpr int kQBlockRows = 128;  // kTileMixQQuantRows
inline constexpr int kKBlockRows = 64;   // kTileMixKQuantRows
inline constexpr int kCellRows = 16;     // kBlockM: routing cell height
inline constexpr int kCellKeys = 32;     // kBlockN: routing cell width

// One side (Q or K) of a quantizer launch. Inputs of head h start at
// x + h * in_head_stride, rows in_row_stride elements apart; outputs are
// contiguous per head.
struct QuantSide {
    const std::uint16_t* x;
    std::int8_t* x8;
    std::uint16_t* scales;
    std::int64_t in_head_stride;
    std::int64_t in_row_stride;
    int rows;
    int block_rows;
    int blocks;  // quantization blocks per head, 0 = side absent
};

// A [heads][rows][d] view, strides in elements, whose heads do not overlap:
// rows are at least d apart, and heads either follow one another (each head
// fits below the next head's start) or interleave inside every row (all
// heads' d elements fit in one row stride, e.g. a [rows][heads][d] tensor).
inline bool strided_heads_ok(int heads, int rows, int d, std::int64_t head_stride, std::int64_t row_stride) {
    if (row_stride < d) return false;
    if (heads <= 1) return true;
    const std::int64_t extent = static_cast<std::int64_t>(rows - 1) * row_stride + d;
    if (head_stride >= extent) return true;
    return head_stride >= d && static_cast<std::int64_t>(heads - 1) * head_stride + d <= row_stride;
}

QuantSide make_quant_side(const std::uint16_t* x, std::int8_t* x8, std::uint16_t* scales,
                          std::int64_t head_stride, int rows, int block_rows, std::int64_t row_stride);

hipError_t launch_quantize(const QuantSide& q, const QuantSide& k, int heads, int d,
                           hipStream_t stream);

}  // namespace tilemix
