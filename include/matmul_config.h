#pragma once
// Tile constants of the TileMix API (reference: include/matmul_config.h:3-14).
//
// These are API constants, not a description of the gfx950 kernel's launch
// geometry: kBlockM x kBlockN (16 query rows x 32 keys) is the routing cell of
// TileMixRouting, the unit the score_dots / decoded_bits traces are defined on,
// and an input of the shared-memory sizing helpers in attention_fused.h. The
// MI355X kernel runs 256-thread workgroups of four 64-lane wavefronts over
// 128x64 tiles and maps each routing cell onto whole 16x16 MFMA blocks, so the
// values below keep their reference meaning unchanged.

inline constexpr int kBlockM = 16;
inline constexpr int kBlockN = 32;
inline constexpr int kTileK = 16;
inline constexpr int kThreads = 64;
inline constexpr int kWarpSize = 32;

static_assert(kBlockM == 16 && kTileK == 16,
              "routing cells are 16 query rows tall and features are padded to 16");
static_assert(kBlockN > 0 && kBlockN % 16 == 0,
              "a routing cell spans whole 16-key column blocks");
static_assert(kWarpSize == 32 && kThreads == (kBlockN / 16) * kWarpSize,
              "reference sizing: one 32-lane group per 16 key columns");
