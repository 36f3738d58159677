#pragma once
// Definitions of the attention kernel (attention.hip) kept apart from it:
// launch parameters, LDS tile movement helpers and block mapping.

#include "tilemix_capi.h"
#include "tilemix_device.h"
#include "tilemix_launch.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tilemix {

inline constexpr float kLog2e = 1.4426950408889634f;
inline constexpr int kXcds = 8;                               // MI355X: 8 XCDs, workgroups dealt round-robin
inline constexpr std::uint32_t kBufferFlags = 0x00020000u;    // raw buffer resource word 3, gfx9 family
inline constexpr int kOutOfRange = static_cast<int>(0x80000000u);  // buffer offset that reads as zero
inline constexpr int kTileKeys = 64;                          // key tile = one K quantization block

// Online-softmax scores enter as x * c (log2 domain) against a reference
// maximum m that is raised lazily - only when a tile's maximum exceeds it by
// more than kLazyRescale (log2 units) - so most tiles skip the O rescale;
// probabilities stay <= 2^kLazyRescale, far inside fp16 range. Every
// probability and the running sum use the same m, so the common factor
// cancels exactly in O = sum(p v) / sum(p).
inline constexpr float kLazyRescale = 8.0f;

struct AttnParams {
    const std::uint16_t* Q;
    const std::uint16_t* K;
    const std::uint16_t* V;
    void* O;  // element type by o_dtype
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
    // Elements between consecutive rows of one head (>= d; d = dense rows).
    std::int64_t q_row;
    std::int64_t k_row;
    std::int64_t v_row;
    std::int64_t o_row;
    std::int64_t words_per_row;
    std::int64_t words_per_head;
    int heads;
    int M;
    int N;
    int d;
    int key_tiles_per_group;
    int group_shift;  // log2(key_tiles_per_group) when that is a power of two, else -1
    int q_tiles16;
    int key_tiles32;
    int q_blocks;
    int k_blocks;
    int causal;
    int fuse_q_quant;
    int int8_operands;
    int o_dtype;  // TILEMIX_DTYPE_F32 / _F16 / _BF16
    float score_log2;  // score_scale * log2(e)
    float score_scale;
    // Key-range split (splits > 1): workgroup b takes tiles [s * split_tiles,
    // (s + 1) * split_tiles) of item b / splits (s = b % splits) and writes
    // its unnormalised O rows to part_o ([splits][M][d] fp32) and its row
    // maximum and sum (log2 domain) to part_ml ([splits][M][2]) instead of O.
    int splits;
    int split_tiles;
    float* part_o;
    float* part_ml;
    // > 0: the workgroups one XCD holds at once (its slots). A head whose
    // query blocks span several rounds of that many workgroups streams its
    // K / V once per round; a workgroup of an odd round walks its key tiles
    // last to first, so it starts on the tiles the round before it left in
    // the XCD's L2. 0: every workgroup walks first to last.
    int reverse_slots;
};

__device__ __forceinline__ half8 concat(half4 a, half4 b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// v_max3_f32 as inline assembly: fmaxf makes the compiler canonicalise every
// operand first (one extra v_max per value); the operands here are scores,
// finite or -inf, never NaN.
__device__ __forceinline__ float max3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Cross-lane exchange without LDS: with a == b == x on entry,
// v_permlane32_swap leaves a = x of the lower half in both halves and b = x
// of the upper half, so max(a, b) or a + b combines lanes l and l ^ 32.
// Inline assembly because the compiler builtin for this swap gets folded as
// if both results were the same value; s_nop 1 covers the VALU-write ->
// permlane-read hazard.
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}


// ds_read_b64_tr_b16: within each 16-lane group, element e of lane i comes
// from lane 4e + i / 4, element i % 4 of that lane's 8-byte row piece.
__device__ __forceinline__ half4 read_tr16(const unsigned char* lds_byte_address) {
    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lds_byte_address));
    return __builtin_bit_cast(half4, raw);
}

// Raw buffer resource (gfx9 layout) held in four SGPRs: base address,
// stride 0, `bytes` records (offsets at or past it read as zero), flags.
__device__ __forceinline__ int4v make_rsrc(const void* base, int bytes) {
    const unsigned long long address = reinterpret_cast<unsigned long long>(base);
    return int4v{__builtin_amdgcn_readfirstlane(static_cast<int>(address & 0xffffffffu)),
                 __builtin_amdgcn_readfirstlane(static_cast<int>((address >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane(bytes), static_cast<int>(kBufferFlags)};
}

// The same buffer viewed from byte `offset` on (0 <= offset < the range):
// base + offset, range - offset. The range check covers the per-lane offset
// only (the scalar offset of a buffer load is not range-checked on gfx9
// family parts), so a tile whose rows run past the end of a head is
// addressed through a view that starts at the tile: its rows past the end
// then fail the check and read as zero instead of reading past the head.
__device__ __forceinline__ int4v rsrc_from(int4v rsrc, int offset) {
    const unsigned long long base = static_cast<unsigned>(rsrc[0]) |
                                    (static_cast<unsigned long long>(static_cast<unsigned>(rsrc[1]) & 0xffffu) << 32);
    const unsigned long long moved = base + static_cast<unsigned>(offset);
    return int4v{static_cast<int>(moved & 0xffffffffu), static_cast<int>((moved >> 32) & 0xffffu),
                 rsrc[2] - offset, rsrc[3]};
}

// LDS byte address of a workgroup-shared buffer, for M0 of an LDS DMA. The
// cast from a generic pointer carries a null check (two scalar instructions),
// so kernels convert each buffer's base once and add offsets to the result.
__device__ __forceinline__ unsigned lds_address_of(const void* shared) {
    return __builtin_amdgcn_readfirstlane(static_cast<unsigned>(
        reinterpret_cast<unsigned long long>((__attribute__((address_space(3))) const void*)(shared))));
}

// 16 bytes per lane from buffer offset soffset + voffset into LDS at byte
// address lds_address + 16 * lane (lds_address is wave-uniform; M0 carries
// it). Issued as inline assembly so that the compiler does not treat it as an
// LDS store: it would otherwise wait for every outstanding tile load before
// any later LDS read it cannot prove disjoint. The kernels order these loads
// themselves - s_waitcnt vmcnt, then a workgroup barrier, before any read of
// the tile.
__device__ __forceinline__ void load_to_lds(int4v rsrc, unsigned lds_address, int voffset, int soffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_address), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory");
}

// bf16 bits of x, rounded to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ std::uint16_t float_to_bf16_bits(float x) {
    const std::uint32_t u = __builtin_bit_cast(std::uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<std::uint16_t>((u >> 16) | 0x40u);
    return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Stores four consecutive outputs of one row at element `offset` of `base`
// in the output type (fp32, or fp16 / bf16 rounded to nearest even); only
// the first `valid` (may be <= 0) are written. `vector`: the row is 16-byte
// aligned and valid >= 4 whenever valid > 0.
__device__ __forceinline__ void store_output(unsigned char* base, int dtype, std::int64_t offset, float4v value,
                                             int valid, bool vector) {
    if (valid <= 0) return;
    if (dtype == TILEMIX_DTYPE_F32) {
        float* out = reinterpret_cast<float*>(base) + offset;
        if (vector) {
            *reinterpret_cast<float4v*>(out) = value;
        } else {
            for (int r = 0; r < 4 && r < valid; ++r) out[r] = value[r];
        }
        return;
    }
    std::uint16_t bits[4];
    for (int r = 0; r < 4; ++r)
        bits[r] = dtype == TILEMIX_DTYPE_F16 ? __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(value[r]))
                                             : float_to_bf16_bits(value[r]);
    std::uint16_t* out = reinterpret_cast<std::uint16_t*>(base) + offset;
    if (vector) {
        *reinterpret_cast<uint2v*>(out) = uint2v{bits[0] | (static_cast<std::uint32_t>(bits[1]) << 16),
                                                 bits[2] | (static_cast<std::uint32_t>(bits[3]) << 16)};
    } else {
        for (int r = 0; r < 4 && r < valid; ++r) out[r] = bits[r];
    }
}

// A 16-bit value at a wave-uniform address, read with s_load_dword (the
// containing aligned dword) and waited on with lgkmcnt: a vector load here
// would be waited on with vmcnt and so also wait for the tile loads above.
__device__ __forceinline__ std::uint16_t load_uniform_u16(const std::uint16_t* address) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(address);
    const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a & ~3ull));
    const unsigned hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a >> 32));
    const unsigned long long word_address = (static_cast<unsigned long long>(hi) << 32) | lo;
    unsigned word;
    // Early clobber: the destination must not share registers with the address.
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=&s"(word) : "s"(word_address) : "memory");
    return static_cast<std::uint16_t>((a & 2) ? (word >> 16) : (word & 0xffffu));
}

// Offset of lane `lane`'s 16-byte piece of wave load `w` of a tile whose LDS
// rows are `lds_stride` bytes apart: its row and 16-byte column follow from
// where it lands (lds offset 1024 w + 16 lane). Padding slots and columns at
// or beyond `row_bytes` (the valid bytes of a global row) read as zero.
__device__ __forceinline__ int lane_offset(int w, int lane, int lds_stride, int row_bytes, int global_row_bytes) {
    const int landing = 1024 * w + 16 * lane;
    const int row = landing / lds_stride;
    const int column = landing - row * lds_stride;
    return column < row_bytes ? row * global_row_bytes + column : kOutOfRange;
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left unconstrained).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier ordering LDS only: waits for this wave's LDS operations,
// not for its vector-memory loads.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Issue priority of this wave against the other waves of its SIMD, set at
// this point of the instruction stream (the compiler moves nothing across).
template <int kLevel>
__device__ __forceinline__ void set_priority() {
    static_assert(kLevel >= 0 && kLevel <= 3, "s_setprio range");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(kLevel);
    __builtin_amdgcn_sched_barrier(0);
}

// Workgroup index -> (head, row group). Workgroups are dealt round-robin to
// the XCDs; all row groups of a head run on one XCD so that its K / V / K8
// stay in that XCD's L2. Causal problems take an XCD's heads four at a time
// (fewer heads' K / V live in its L2 at once) and start the heaviest (last)
// row groups of those heads first, head after head, to shorten the tail.
__device__ __forceinline__ void map_block(int linear, int heads, int groups, bool causal, int& head, int& group) {
    int slot_group;
    if (heads % kXcds == 0) {
        const int xcd = linear % kXcds, slot = linear / kXcds;
        const int heads_per_xcd = heads / kXcds;
        if (causal) {
            const int batch_heads = heads_per_xcd % 4 == 0 ? 4 : heads_per_xcd;
            const int per_batch = batch_heads * groups;
            const int batch = slot / per_batch, r = slot % per_batch;
            head = xcd + kXcds * (batch * batch_heads + r % batch_heads);
            slot_group = r / batch_heads;
        } else {
            head = xcd + kXcds * (slot / groups);
            slot_group = slot % groups;
        }
    } else if (causal) {
        head = linear % heads;
        slot_group = linear / heads;
    } else {
        head = linear / groups;
        slot_group = linear % groups;
    }
    group = causal ? groups - 1 - slot_group : slot_group;
}

// Whether workgroup `linear` (dealt to XCD linear % kXcds) runs in an odd
// round of `reverse_slots` workgroups on its XCD (AttnParams::reverse_slots).
__device__ __forceinline__ bool reversed_round(int linear, int reverse_slots) {
    return reverse_slots > 0 && ((linear / kXcds / reverse_slots) & 1) != 0;
}

}  // namespace tilemix
