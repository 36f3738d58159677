#pragma once
// TileMix public C++ API on HIP for MI355X (gfx950).
//
// Same names, constants, sizing helpers, structs and entry points as the
// reference header (include/attention_fused.h:11-72); the CUDA types become
// their HIP counterparts (hipError_t, hipStream_t, __half). The two entry
// points are inline wrappers over the C ABI in tilemix_capi.h, implemented in
// libtilemix_hip.so.

#include "matmul_config.h"
#include "tilemix_capi.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

inline constexpr int kFusedMaxHeadDim = 128;
inline constexpr int kFusedRowThreads = kThreads / kBlockM;
inline constexpr int kTileMixQQuantRows = 128;
inline constexpr int kTileMixKQuantRows = 64;
static_assert(kTileMixQQuantRows % kBlockM == 0 && kTileMixKQuantRows % kBlockN == 0);
static_assert(kThreads % kBlockM == 0 && kThreads % kWarpSize == 0);
static_assert(kFusedRowThreads > 0 && kFusedRowThreads <= kWarpSize &&
              (kFusedRowThreads & (kFusedRowThreads - 1)) == 0);
static_assert(kBlockN % kFusedRowThreads == 0 && kFusedMaxHeadDim % kFusedRowThreads == 0);

// Reference-defined workspace sizes (attention_fused.h:21-32). The MI355X
// kernel uses its own, larger LDS layout; these helpers keep their reference
// values because callers and tests use them as API facts.
inline constexpr std::size_t fused_fp16_shared_bytes(int d) {
    if (d <= 0 || d > kFusedMaxHeadDim) return 0;
    const int padded_d = ((d + kTileK - 1) / kTileK) * kTileK;
    return sizeof(__half) * static_cast<std::size_t>(padded_d) * (kBlockM + 2 * kBlockN)
         + sizeof(float) * kBlockM * kBlockN;
}

inline constexpr std::size_t tilemix_shared_bytes(int d, bool quantized) {
    if (d <= 0 || d > kFusedMaxHeadDim) return 0;
    const int padded_d = ((d + kTileK - 1) / kTileK) * kTileK;
    return fused_fp16_shared_bytes(d) + (quantized ? (kBlockM + kBlockN) * padded_d : 0);
}

// Routing-mask footprint (attention_fused.h:34-45): one bit per group of
// key_tiles_per_group 32-key tiles, 64 groups per word, one word row per
// 16-row query tile.
inline constexpr std::size_t tilemix_routing_words_per_row(int N, int key_tiles_per_group) {
    if (N <= 0 || key_tiles_per_group <= 0) return 0;
    const std::size_t key_tiles = (static_cast<std::size_t>(N) - 1) / kBlockN + 1;
    const std::size_t groups = (key_tiles - 1) / key_tiles_per_group + 1;
    return (groups - 1) / 64 + 1;
}

inline constexpr std::size_t tilemix_routing_word_count(int M, int N, int key_tiles_per_group) {
    if (M <= 0) return 0;
    return ((static_cast<std::size_t>(M) - 1) / kBlockM + 1)
         * tilemix_routing_words_per_row(N, key_tiles_per_group);
}

// attention_fused.h:47-52: bit 1 = INT8 scores, 0 = FP16 scores.
struct TileMixRouting {
    const std::uint64_t* words = nullptr;
    std::size_t word_count = 0;
    int key_tiles_per_group = 1;
    std::uint8_t* decoded_bits = nullptr;
};

// attention_fused.h:54-60: quantize_tilemix_qk outputs plus the optional
// int32 score trace.
struct TileMixQuantized {
    const std::int8_t* q = nullptr;
    const std::int8_t* k = nullptr;
    const __half* q_scales = nullptr;
    const __half* k_scales = nullptr;
    std::int32_t* score_dots = nullptr;
};

inline hipError_t quantize_tilemix_qk(const __half* Q, const __half* K,
                                      std::int8_t* Q8, std::int8_t* K8,
                                      __half* q_scales, __half* k_scales,
                                      int M, int N, int d, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(tilemix_quantize_qk(
        reinterpret_cast<const std::uint16_t*>(Q), reinterpret_cast<const std::uint16_t*>(K),
        Q8, K8, reinterpret_cast<std::uint16_t*>(q_scales),
        reinterpret_cast<std::uint16_t*>(k_scales), M, N, d, stream));
}

inline hipError_t launch_fused_fp16_attention(const __half* Q, const __half* K, const __half* V,
                                              float* O, int M, int N, int d, float score_scale,
                                              hipStream_t stream = nullptr,
                                              const TileMixRouting& routing = {},
                                              const TileMixQuantized& quantized = {}) {
    return static_cast<hipError_t>(tilemix_attention(
        reinterpret_cast<const std::uint16_t*>(Q), reinterpret_cast<const std::uint16_t*>(K),
        reinterpret_cast<const std::uint16_t*>(V), O, M, N, d, score_scale, stream,
        routing.words, routing.word_count, routing.key_tiles_per_group, routing.decoded_bits,
        quantized.q, quantized.k, reinterpret_cast<const std::uint16_t*>(quantized.q_scales),
        reinterpret_cast<const std::uint16_t*>(quantized.k_scales), quantized.score_dots));
}
