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
// x + h * in_head_stride; outputs are contiguous per head.
struct QuantSide {
    const std::uint16_t* x;
    std::int8_t* x8;
    std::uint16_t* scales;
    std::int64_t in_head_stride;
    int rows;
    int block_rows;
    int blocks;  // quantization blocks per head, 0 = side absent
};

QuantSide make_quant_side(const std::uint16_t* x, std::int8_t* x8, std::uint16_t* scales,
                          std::int64_t head_stride, int rows, int block_rows);

hipError_t launch_quantize(const QuantSide& q, const QuantSide& k, int heads, int d,
                           hipStream_t stream);

}  // namespace tilemix
