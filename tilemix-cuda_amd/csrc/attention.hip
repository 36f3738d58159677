// Routed INT8/FP16 fused attention for gfx950 (MI355X).
//
// Replaces fused_fp16_attention + launch_fused_fp16_attention of the reference
// (src/tilemix.cu:51-220, 238-278). Design (not a translation):
//
//  * A 256-thread workgroup (4 wave64s) owns 128 query rows of one head - one
//    Q quantization block - and streams the keys in 64-key tiles, one K
//    quantization block each, so q_scale is constant per workgroup and
//    k_scale per tile.
//  * Each wave owns 32 query rows (two 16-row routing cells tall) and works
//    on 32x32 MFMA blocks. Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_f16 (FP16 cells) or v_mfma_i32_32x32x32_i8 (INT8
//    cells, exact int32 dots), one block per 32 keys. In that layout lane
//    (q, h) = (lane % 32, lane / 32) holds 16 keys of query row q, so a row's
//    online-softmax state lives in lanes q and q + 32 and its maximum needs
//    one cross-lane step. A 32x32 MFMA does the work of two 16x16 ones but
//    holds the wave's instruction issue about as long as one, which leaves
//    the SIMD free for the other wave's (or this wave's) VALU work.
//  * The probabilities stay in registers and feed O^T += V^T P^T on
//    v_mfma_f32_32x32x16_f16: the accumulator elements of 8 consecutive
//    score slots are exactly the P^T operand of one 16-key step, and the V^T
//    operand is read from the row-major V tile in LDS with
//    ds_read_b64_tr_b16, which transposes 16-bit elements across each
//    16-lane group (key order inside a step permuted identically on both
//    operands). Row sums add exactly the fp16 probabilities P.V uses
//    (v_dot2_f32_f16 against ones); the two lanes of a row are summed once,
//    at the end.
//  * K, K8 and V tiles move HBM -> LDS with buffer_load ... lds (no VGPR
//    staging): per-lane offsets into the LDS rows (unpadded with rotated
//    16-byte chunks: all K8 rows, K / V rows of 128 or 256 bytes) are
//    computed once, each tile only changes a scalar offset, and rows past
//    the end of the head read as zero. Every wave issues the same number of
//    loads per buffer (spare slots read out of range into a 1 KiB landing
//    area), so the issue code has no branches. V has two buffers, K and K8
//    one each: the next tile's K, K8 and V are all fetched after the tile's
//    second barrier, while softmax and P.V run, so no tile load is issued
//    among the score MFMAs; two barriers per tile. At d = 128, 56 KiB of tile
//    buffers per workgroup.
//  * Each SIMD runs one wave of each of the CU's two workgroups. A tile is an
//    MFMA phase (P.V, barrier, next scores) and a VALU phase (softmax). A
//    wave's issue priority is low in the first half of each phase and high
//    in the second, so of two waves in the same phase the one further along
//    wins arbitration and leaves it first: this pushes the pair apart, one
//    on the matrix core while the other runs exponentials.
//  * A 32-key MFMA block is one routing cell wide and two cells (the wave's
//    two 16-row halves) tall. The branch is taken on wave-uniform route
//    masks; a wave whose cells mix routes computes both score kinds and
//    selects per lane.
//  * The optional in-kernel Q quantization reproduces quantize_tilemix_qk's
//    bytes exactly: the workgroup's 128 rows are exactly one Q block. The
//    bytes reach the INT8 operand layout through a lane swap between the
//    two halves of the wave, not through LDS.

#include "attention_common.h"
#include "tilemix_capi.h"

#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>

namespace tilemix {
namespace {

constexpr int kThreadsPerGroup = 256;
constexpr int kWavesPerGroup = kThreadsPerGroup / kWave;
constexpr int kRowsPerGroup = 128;  // one Q quantization block
constexpr int kRowsPerWave = 32;
#ifndef TILEMIX_GROUPS_PER_CU
#define TILEMIX_GROUPS_PER_CU 2
#endif
// Workgroups per CU the register allocation is sized for (launch bound).
constexpr int kGroupsPerCU = TILEMIX_GROUPS_PER_CU;

template <int DC>
struct Layout {
    static constexpr int kDP = 32 * DC;            // padded head dim, fp16 path
    static constexpr int kD8C = (DC + 1) / 2;      // 64-feature chunks, int8 path
    static constexpr int kDP8 = 64 * kD8C;
    // K / V rows hold 2 * kDP bytes. Rows of 256 bytes (d > 96) and 128 bytes
    // (32 < d <= 64) are unpadded, with 16-byte chunk c of row r at chunk
    // position (c + rot(r)) mod (chunks per row), so that the fragment reads
    // are free of LDS bank conflicts with no pad bytes to move (rot below).
    // Other rows are padded by 16 (K) or 32 (V) bytes. K8 rows are 128 bytes
    // (d > 64) or 64 bytes, rotated the same way.
    static constexpr int kRowBytes = kDP * 2;
    static constexpr bool kRotate = kRowBytes == 256 || kRowBytes == 128;
    static constexpr bool kRotate8 = kDP8 == 128 || kDP8 == 64;
    static constexpr int kKStride = kRotate ? kRowBytes : kRowBytes + 16;
    static constexpr int kVStride = kRotate ? kRowBytes : kRowBytes + 32;
    static constexpr int kK8Stride = kRotate8 ? kDP8 : kDP8 + 16;
    static constexpr int kKBytes = kTileKeys * kKStride;
    static constexpr int kVBytes = kTileKeys * kVStride;
    static constexpr int kK8Bytes = kTileKeys * kK8Stride;
    // One buffer_load ... lds per wave moves 1 KiB (64 lanes x 16 bytes).
    static constexpr int kKLoads = kKBytes / 1024;
    static constexpr int kVLoads = kVBytes / 1024;
    static constexpr int kK8Loads = kK8Bytes / 1024;
    static constexpr int kKPerWave = (kKLoads + kWavesPerGroup - 1) / kWavesPerGroup;
    static constexpr int kVPerWave = (kVLoads + kWavesPerGroup - 1) / kWavesPerGroup;
    static constexpr int kK8PerWave = (kK8Loads + kWavesPerGroup - 1) / kWavesPerGroup;
    // K, V buffer 0, K8, V buffer 1.
    static constexpr int kV1Offset = kVBytes + kK8Bytes;  // V buffer 1 - V buffer 0
    static constexpr int kSmemBytes = kKBytes + kVBytes + kK8Bytes + kVBytes;
    static_assert(kKBytes % 1024 == 0 && kVBytes % 1024 == 0 && kK8Bytes % 1024 == 0,
                  "tiles are whole wave loads");
    // Chunk rotation of a rotated row of kChunks 16-byte chunks. Key rows
    // (K, K8) are read as 32 consecutive rows x one chunk per half-wave: the
    // rows that share one 256-byte sweep of the banks share a rotation, and
    // consecutive sweeps step it by one chunk (measured on 64-byte K8 rows:
    // 13 % of LDS-active cycles in bank conflicts with a rotation that steps
    // every two rows, 0.9 % with this one). Value rows are read by
    // ds_read_b64_tr_b16 in 4-row x 16-feature blocks.
    template <int kChunks, bool kKey>
    __device__ static int rot(int row) {
        static_assert(kChunks == 16 || kChunks == 8 || kChunks == 4, "rotated rows are 256, 128 or 64 bytes");
        if constexpr (kKey)
            return kChunks == 16 ? row & 15 : kChunks == 8 ? (row >> 1) & 7 : (row >> 2) & 3;
        else
            return kChunks == 16 ? (2 * row) & 15 : kChunks == 8 ? row & 6 : 2 * ((row >> 2) & 1);
    }
    // Offset of byte `byte` of row `row` in a rotated tile.
    template <int kChunks, bool kKey>
    __device__ static int rotated(int row, int byte) {
        return row * 16 * kChunks + ((((byte >> 4) + rot<kChunks, kKey>(row)) & (kChunks - 1)) << 4) + (byte & 15);
    }
    // Global offset that DMA lane `lane` of 1 KiB piece w fetches for a
    // rotated tile (kOutOfRange past the row's bytes): the inverse of rotated.
    template <int kChunks, bool kKey>
    __device__ static int rotated_lane(int w, int lane, int row_bytes, int global_row_bytes) {
        const int landing = 1024 * w + 16 * lane;
        const int row = landing / (16 * kChunks);
        const int column = ((((landing >> 4) & (kChunks - 1)) - rot<kChunks, kKey>(row)) & (kChunks - 1)) << 4;
        return column < row_bytes ? row * global_row_bytes + column : kOutOfRange;
    }
    // Offset of byte `byte` (< 2 * kDP, or < kDP8 for K8) of row `row` in the
    // K / V / K8 tile.
    __device__ static int k_at(int row, int byte) {
        if constexpr (kRotate) return rotated<kRowBytes / 16, true>(row, byte);
        else return row * kKStride + byte;
    }
    __device__ static int v_at(int row, int byte) {
        if constexpr (kRotate) return rotated<kRowBytes / 16, false>(row, byte);
        else return row * kVStride + byte;
    }
    __device__ static int k8_at(int row, int byte) {
        if constexpr (kRotate8) return rotated<kDP8 / 16, true>(row, byte);
        else return row * kK8Stride + byte;
    }
    // Global offset that DMA lane `lane` of 1 KiB piece w fetches.
    template <bool kKey>
    __device__ static int kv_lane_offset(int w, int lane, int stride, int row_bytes, int global_row_bytes) {
        if constexpr (kRotate) return rotated_lane<kRowBytes / 16, kKey>(w, lane, row_bytes, global_row_bytes);
        else return lane_offset(w, lane, stride, row_bytes, global_row_bytes);
    }
    __device__ static int k8_lane_offset(int w, int lane, int row_bytes) {
        if constexpr (kRotate8) return rotated_lane<kDP8 / 16, true>(w, lane, row_bytes, row_bytes);
        else return lane_offset(w, lane, kK8Stride, row_bytes, row_bytes);
    }
};

typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int16v __attribute__((ext_vector_type(16)));

// Online-softmax state of the query row a lane owns (row lane & 31 of the
// wave's 32; lanes l and l ^ 32 hold the same row, each for half of every
// 32-key block), scores in the log2 domain, m raised lazily (kLazyRescale).
template <int kOB>
struct RowState {
    // O^T accumulators: o[fb][j] is output row R = 8 (j / 4) + 4 h + j % 4
    // (h = lane / 32) of feature block fb, i.e. feature 16 fb + R for R < 16
    // and kDP / 2 + 16 fb + R - 16 above (the two 16-row halves of a block
    // sit kDP / 2 features apart, which keeps the transposed V reads free of
    // bank conflicts).
    float16v o[kOB];
    float lsum;       // this lane's part of the row sum of P (the fp16 values P.V uses)
    float m;
};

// Maximum of the 16 values of a 32x32 accumulator block, 8 v_max3.
__device__ __forceinline__ float block_max16(const float16v& x) {
    const float a = max3(x[0], x[1], x[2]), b = max3(x[3], x[4], x[5]), e = max3(x[6], x[7], x[8]);
    const float f = max3(x[9], x[10], x[11]), g = max3(x[12], x[13], x[14]);
    return max3(max3(a, b, e), max3(f, g, x[15]), x[15]);
}

// x[kb][j] holds the score of the lane's row against key 32 kb + 8 (j / 4) +
// 4 h + j % 4; c is the per-tile log2-domain factor (>= 0; explicit scores
// pass c = 1). ph[ks] / pl[ks] receive the fp16 probabilities of keys
// 16 ks + {4h .. 4h + 3, 8 + 4h .. 8 + 4h + 3}: the B operand (P^T) of the
// 32x32x16 P.V MFMA for key step ks.
template <int kOB, bool kPrecise>
__device__ __forceinline__ void softmax_tile(RowState<kOB>& st, const float16v (&x)[2], float c,
                                             half8 (&ph)[4], half8 (&pl)[4]) {
    const float tile = max3(block_max16(x[0]), block_max16(x[1]), block_max16(x[1])) * c;  // c >= 0
    // The row's maximum exceeds m + kLazyRescale exactly when one of its two
    // lanes' own maxima does.
    if (__any(tile > st.m + kLazyRescale)) {
        float a = tile, b = tile;
        permlane32_swap(a, b);
        const float m_new = fmaxf(st.m, max3(a, b, b));
        // Rows with no visible key yet keep m = -inf (their sums are still 0).
        const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(st.m - m_new);
        st.m = m_new;
#pragma unroll
        for (int fb = 0; fb < kOB; ++fb) st.o[fb] *= alpha;
        st.lsum *= alpha;
    }
    // m == -inf only while every score seen, this tile included, is masked.
    const float neg_m = st.m == -INFINITY ? 0.0f : -st.m;
    const half2v ones{1.0f16, 1.0f16};
    float part[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int kb = ks >> 1, base = 8 * (ks & 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kb][base + e], c, neg_m));
            const _Float16 hv = static_cast<_Float16>(v);
            ph[ks][e] = hv;
            if constexpr (kPrecise) pl[ks][e] = static_cast<_Float16>(v - static_cast<float>(hv));
        }
        // Row sums of exactly the fp16 values the P.V MFMAs use.
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            sum = __builtin_amdgcn_fdot2(half2v{ph[ks][e], ph[ks][e + 1]}, ones, sum, false);
            if constexpr (kPrecise) sum = __builtin_amdgcn_fdot2(half2v{pl[ks][e], pl[ks][e + 1]}, ones, sum, false);
        }
        part[ks] = sum;
        if (ks == 1) set_priority<2>();  // second half of the VALU phase
    }
    st.lsum += (part[0] + part[1]) + (part[2] + part[3]);
}

// load_to_lds with M0 = lds_address + kOffset, the add issued inside the asm
// so that the compiler keeps one scalar address per buffer, not one per slot.
template <int kOffset>
__device__ __forceinline__ void load_to_lds_at(int4v rsrc, unsigned lds_address, int voffset, int soffset) {
    if constexpr (kOffset == 0) {
        load_to_lds(rsrc, lds_address, voffset, soffset);
    } else {
        asm volatile("s_add_u32 m0, %0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :
                     : "s"(lds_address), "v"(voffset), "s"(rsrc), "s"(soffset), "i"(kOffset)
                     : "memory", "scc");
    }
}

// The 1 KiB pieces one wave moves of a tile buffer that splits evenly over
// the workgroup's four waves: slot t lands 4 KiB past slot t - 1 (pieces
// wave, wave + 4, ...), so all slots share the first one's LDS address.
template <int t, int kSlots>
__device__ __forceinline__ void load_slots_from(int4v rsrc, unsigned first, const int (&voffset)[kSlots], int soffset) {
    if constexpr (t < kSlots) {
        load_to_lds_at<4096 * t>(rsrc, first, voffset[t], soffset);
        load_slots_from<t + 1, kSlots>(rsrc, first, voffset, soffset);
    }
}
template <int kSlots>
__device__ __forceinline__ void load_slots(int4v rsrc, unsigned first, const int (&voffset)[kSlots], int soffset) {
    load_slots_from<0, kSlots>(rsrc, first, voffset, soffset);
}

// kSplit: the workgroup covers one range of key tiles of its 128-row block
// and writes that range's partial row state (AttnParams::splits); only the
// per-head entry point launches it.
template <int DC, bool kVector, bool kPrecise, bool kDots, bool kSplit>
__global__ __launch_bounds__(kThreadsPerGroup, kGroupsPerCU) void attention_kernel(const AttnParams p) {
    using L = Layout<DC>;
    constexpr int kDP = L::kDP;
    constexpr int kOB = DC;               // 32-feature output blocks
    constexpr int kQC = kDP / 16;         // 16-feature Q / K chunks (fp16 MFMA k-steps)
    constexpr int kQ8C = L::kDP8 / 32;    // 32-feature Q8 / K8 chunks (int8 MFMA k-steps)
    __shared__ __attribute__((aligned(16))) unsigned char smem[L::kSmemBytes];
    __shared__ unsigned group_bits[kWavesPerGroup];
    // Landing area of the spare DMA slots (written with zeros, never read).
    __shared__ __attribute__((aligned(16))) unsigned char lds_spare[1024];
    unsigned char* const lds_k = smem;
    unsigned char* const lds_v = smem + L::kKBytes;
    unsigned char* const lds_k8 = smem + L::kKBytes + L::kVBytes;
    // LDS byte addresses of the tile buffers (M0 of the tile DMA), converted once.
    const unsigned lds_k_address = lds_address_of(smem);
    const unsigned lds_v_address = lds_k_address + L::kKBytes;
    const unsigned lds_k8_address = lds_v_address + L::kVBytes;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15;
    const int q = lane & 31;  // the lane's query row within the wave (and its MFMA column)
    const int h = lane >> 5;  // which half of each 32-key / 16-feature block the lane holds

    int head32, qblock;
    int item = blockIdx.x, split = 0;
    if constexpr (kSplit) {
        item = blockIdx.x / p.splits;
        split = blockIdx.x - item * p.splits;
    }
    map_block(item, p.heads, p.q_blocks, p.causal != 0, head32, qblock);
    const std::int64_t head = head32;
    const int q0 = qblock * kRowsPerGroup;
    const int qw = q0 + wave * kRowsPerWave;
    const int M = p.M, N = p.N, d = p.d;

    const std::uint16_t* Qh = p.Q + head * p.q_stride;
    const std::uint16_t* Kh = p.K + head * p.k_stride;
    const std::uint16_t* Vh = p.V + head * p.v_stride;
    const std::int8_t* K8h = p.K8 + head * static_cast<std::int64_t>(N) * d;
    unsigned char* const Oh = static_cast<unsigned char*>(p.O) + head * p.o_stride * (p.o_dtype == TILEMIX_DTYPE_F32 ? 4 : 2);

    // ---------------------------------------------------------------- Q
    // B operand of the 32x32x16 QK^T MFMA: lane (q, h) holds features
    // 16c + 8h .. 16c + 8h + 7 of its row for chunk c.
    half8 qf[kQC];
    {
        const int row = qw + q;
#pragma unroll
        for (int c = 0; c < kQC; ++c) {
            const int feature = 16 * c + 8 * h;
            if constexpr (kVector) {
                qf[c] = (row < M && feature < d)
                    ? *reinterpret_cast<const half8*>(Qh + static_cast<std::int64_t>(row) * p.q_row + feature)
                    : half8{};
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qf[c][e] = (row < M && feature + e < d)
                        ? __builtin_bit_cast(_Float16, Qh[static_cast<std::int64_t>(row) * p.q_row + feature + e])
                        : static_cast<_Float16>(0.0f);
            }
        }
    }

    // The wave's quantized Q rows (B operand of the INT8 MFMA), kept in
    // registers: lane (q, h) holds features 32m + 16h .. 32m + 16h + 15 of
    // its row for chunk m.
    int4v q8f[kQ8C];
    float q_scale = 0.0f;
    if (p.int8_operands) {
        if (p.fuse_q_quant) {
            // The workgroup's rows are exactly one 128-row Q block. Its
            // maximum |x| as fp16 bit patterns: unsigned order is float order
            // for them, NaN patterns (> 0x7c00) sorting above +inf.
            unsigned top = 0;
#pragma unroll
            for (int c = 0; c < kQC; ++c) {
                const uint4v words = __builtin_bit_cast(uint4v, qf[c]);
#pragma unroll
                for (int w = 0; w < 4; ++w) top = max_u16x2(top, words[w] & 0x7fff7fffu);
            }
            unsigned bits = wave_max_bits(max(top & 0xffffu, top >> 16));
            if (lane == 0) group_bits[wave] = bits;
            __syncthreads();
            bits = max(max(group_bits[0], group_bits[1]), max(group_bits[2], group_bits[3]));
            if (bits > 0x7c00u) {
                // A NaN in the block: the maximum skips NaNs, as fmaxf does.
                unsigned clean = 0;
#pragma unroll
                for (int c = 0; c < kQC; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        // The element is copied out first: __builtin_bit_cast
                        // applied to a vector element expression reads
                        // element 0 under this compiler.
                        const _Float16 x = qf[c][e];
                        const unsigned hb = __builtin_bit_cast(std::uint16_t, x) & 0x7fffu;
                        clean = hb <= 0x7c00u ? max(clean, hb) : clean;
                    }
                clean = wave_max_bits(clean);
                __syncthreads();
                if (lane == 0) group_bits[wave] = clean;
                __syncthreads();
                bits = max(max(group_bits[0], group_bits[1]), max(group_bits[2], group_bits[3]));
            }
            const float scale = block_scale(half_bits_to_float(static_cast<std::uint16_t>(bits)));
            const float recip = 1.0f / scale;
            const _Float16 stored = static_cast<_Float16>(scale);
            q_scale = static_cast<float>(stored);
            if (tid == 0 && p.q_scales_out)
                p.q_scales_out[head * p.q_blocks + qblock] = __builtin_bit_cast(std::uint16_t, stored);
            {
                const int row = qw + q;
                // Bytes of fp16 chunk c (features 16c + 8h .. + 7 of the row).
                uint2v packed[L::kDP8 / 16];
#pragma unroll
                for (int c = 0; c < L::kDP8 / 16; ++c) {
                    packed[c] = uint2v{0u, 0u};
                    if (c < kQC && scale > 0.0f) {
                        const uint4v words = __builtin_bit_cast(uint4v, qf[c < kQC ? c : 0]);
                        int v[8];
#pragma unroll
                        for (int w = 0; w < 4; ++w) {
                            v[2 * w] = quantize_half<0>(words[w], scale, recip);
                            v[2 * w + 1] = quantize_half<1>(words[w], scale, recip);
                        }
                        packed[c][0] = pack_bytes(v[0], v[1], v[2], v[3]);
                        packed[c][1] = pack_bytes(v[4], v[5], v[6], v[7]);
                    }
                    const int feature = 16 * c + 8 * h;
                    if (p.q8_out && row < M && feature < d) {
                        std::int8_t* dst = p.q8_out + head * static_cast<std::int64_t>(M) * d +
                                           static_cast<std::int64_t>(row) * d + feature;
                        if constexpr (kVector) {
                            *reinterpret_cast<uint2v*>(dst) = packed[c];
                        } else {
                            for (int e = 0; e < 8 && feature + e < d; ++e)
                                dst[e] = static_cast<std::int8_t>(packed[c][e / 4] >> (8 * (e % 4)));
                        }
                    }
                }
                // INT8 chunk m = fp16 chunks 2m (features 32m .. 32m + 15)
                // and 2m + 1 (32m + 16 .. 32m + 31). Lanes h = 0 keep their
                // bytes of chunk 2m and take lane (q, 1)'s; lanes h = 1 keep
                // their bytes of chunk 2m + 1 and take lane (q, 0)'s: one
                // v_permlane32_swap per dword.
#pragma unroll
                for (int m = 0; m < kQ8C; ++m) {
                    const uint2v keep = h ? packed[2 * m + 1] : packed[2 * m];
                    const uint2v send = h ? packed[2 * m] : packed[2 * m + 1];
                    std::uint32_t got[2];
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const std::uint32_t word = send[k];  // copied out before the bit cast, see above
                        float a = __builtin_bit_cast(float, word), b = a;
                        permlane32_swap(a, b);  // a: lane (q, 0)'s dword, b: lane (q, 1)'s
                        got[k] = __builtin_bit_cast(std::uint32_t, h ? a : b);
                    }
                    q8f[m] = h ? int4v{static_cast<int>(got[0]), static_cast<int>(got[1]), static_cast<int>(keep[0]),
                                       static_cast<int>(keep[1])}
                               : int4v{static_cast<int>(keep[0]), static_cast<int>(keep[1]), static_cast<int>(got[0]),
                                       static_cast<int>(got[1])};
                }
            }
        } else {
            // Q8 rows already come in the operand layout: 16 bytes per lane
            // and chunk, read straight into q8f.
            q_scale = half_bits_to_float(p.q_scales[head * p.q_blocks + qblock]);
            const std::int8_t* Q8h = p.Q8 + head * static_cast<std::int64_t>(M) * d;
            const int row = qw + q;
#pragma unroll
            for (int m = 0; m < kQ8C; ++m) {
                const int feature = 32 * m + 16 * h;
                int4v chunk;
                if constexpr (kVector) {
                    chunk = (row < M && feature < d)
                        ? *reinterpret_cast<const int4v*>(Q8h + static_cast<std::int64_t>(row) * d + feature)
                        : int4v{0, 0, 0, 0};
                } else {
                    unsigned char bytes[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        bytes[e] = (row < M && feature + e < d)
                            ? static_cast<unsigned char>(Q8h[static_cast<std::int64_t>(row) * d + feature + e])
                            : 0;
                    chunk = __builtin_bit_cast(int4v, bytes);
                }
                q8f[m] = chunk;
            }
        }
    }

    // Key tiles are visited first to last, or last to first in a reversed
    // round (AttnParams::reverse_slots; the online softmax takes the tiles in
    // any order).
    const int step = (!kSplit && reversed_round(blockIdx.x, p.reverse_slots)) ? -1 : 1;

    // ------------------------------------------------------ routing masks
    // One pass decodes four tiles: lane 16t + c decodes cell c (row c / 2,
    // key half c % 2) of tile jb + t from the route / skip word it keeps for
    // its query tile; the word is reloaded only when the tile's group moves
    // to another 64-group block. The two 64-bit ballots hold the four tiles'
    // wave-uniform masks, bit 16t + 2r + h <-> tile jb + t, cell (r, h). The
    // pass starts at the tile asked for (jb = j) when the walk goes forward,
    // and ends at it (jb = j - 3) when it goes backward; tiles before the
    // first read as skipped.
    const int qt0 = q0 / 16;
    const int my_qt = qt0 + ((lane & 15) >> 1);
    const bool my_row_valid = my_qt < p.q_tiles16;
    const std::int64_t my_word_base =
        head * p.words_per_head + static_cast<std::int64_t>(my_qt) * p.words_per_row;
    std::int64_t cached_block = -1;
    std::uint64_t cached_route = 0, cached_skip = 0;
    std::uint64_t batch_int8 = 0, batch_skip = 0;
    int batch_first = -4;
    auto tile_masks = [&](int j, std::uint32_t& int8_mask, std::uint32_t& skip_mask) {
        if (static_cast<unsigned>(j - batch_first) >= 4u) {
            batch_first = step < 0 ? j - 3 : j;
            const int kt = 2 * (batch_first + (lane >> 4)) + (lane & 1);
            bool skip = true, int8 = false;
            if (my_row_valid && kt >= 0 && kt < p.key_tiles32) {
                const unsigned group = p.group_shift >= 0 ? static_cast<unsigned>(kt) >> p.group_shift
                                                          : static_cast<unsigned>(kt) / static_cast<unsigned>(p.key_tiles_per_group);
                const std::int64_t block = group >> 6;
                if (block != cached_block) {
                    cached_block = block;
                    cached_route = p.route_words ? p.route_words[my_word_base + block] : 0ull;
                    cached_skip = p.skip_words ? p.skip_words[my_word_base + block] : 0ull;
                }
                const unsigned bit = static_cast<unsigned>(group & 63);
                skip = (cached_skip >> bit) & 1u;
                int8 = !skip && ((cached_route >> bit) & 1u);
            }
            batch_int8 = __ballot(int8);
            batch_skip = __ballot(skip);
        }
        const int shift = 16 * (j - batch_first);
        int8_mask = static_cast<std::uint32_t>(batch_int8 >> shift) & 0xffffu;
        skip_mask = static_cast<std::uint32_t>(batch_skip >> shift) & 0xffffu;
    };

    // ------------------------------------------------------ tile movement
    // Buffer ranges end after the last row's d elements; row strides apart.
    const std::int64_t k_bytes = (static_cast<std::int64_t>(N - 1) * p.k_row + d) * 2;
    const std::int64_t v_bytes = (static_cast<std::int64_t>(N - 1) * p.v_row + d) * 2;
    const int4v rsrc_k = make_rsrc(Kh, static_cast<int>(k_bytes));
    const int4v rsrc_v = make_rsrc(Vh, static_cast<int>(v_bytes));
    const int4v rsrc_k8 = make_rsrc(p.int8_operands ? K8h : p.K8,
                                    static_cast<int>(p.int8_operands ? static_cast<std::int64_t>(N) * d : 0));
    const int k_row_bytes = static_cast<int>(p.k_row * 2), v_row_bytes = static_cast<int>(p.v_row * 2);
    // Each wave issues the same number of DMAs per tile buffer, so the issue
    // code has no branches: slot t of a wave moves 1 KiB piece wave + 4t, and
    // a slot past the buffer's last piece reads out of range (zeros, no
    // memory traffic) into lds_spare.
    const unsigned lds_spare_address = lds_address_of(lds_spare);
    int off_k[L::kKPerWave], off_v[L::kVPerWave], off_k8[L::kK8PerWave];
    unsigned dst_k[L::kKPerWave], dst_v[L::kVPerWave], dst_k8[L::kK8PerWave];
    if constexpr (kVector) {
#pragma unroll
        for (int t = 0; t < L::kKPerWave; ++t) {
            const int w = wave + kWavesPerGroup * t;
            off_k[t] = w < L::kKLoads ? L::template kv_lane_offset<true>(w, lane, L::kKStride, 2 * d, k_row_bytes) : kOutOfRange;
            dst_k[t] = w < L::kKLoads ? lds_k_address + 1024 * w : lds_spare_address;
        }
#pragma unroll
        for (int t = 0; t < L::kVPerWave; ++t) {
            const int w = wave + kWavesPerGroup * t;
            off_v[t] = w < L::kVLoads ? L::template kv_lane_offset<false>(w, lane, L::kVStride, 2 * d, v_row_bytes) : kOutOfRange;
            dst_v[t] = w < L::kVLoads ? lds_v_address + 1024 * w : lds_spare_address;
        }
#pragma unroll
        for (int t = 0; t < L::kK8PerWave; ++t) {
            const int w = wave + kWavesPerGroup * t;
            off_k8[t] = w < L::kK8Loads ? L::k8_lane_offset(w, lane, d) : kOutOfRange;
            dst_k8[t] = w < L::kK8Loads ? lds_k8_address + 1024 * w : lds_spare_address;
        }
    }
    // Tile DMA of one buffer: every slot of this wave from resource r at
    // scalar offset soffset. A tile that runs past the last key (the head's
    // last tile when N % 64 != 0) is issued through a view starting at the
    // tile (rsrc_from), so that its rows past N fail the range check.
    auto k_slots = [&](int4v r, int soffset) {
        if constexpr (L::kKLoads % kWavesPerGroup == 0) {
            load_slots(r, dst_k[0], off_k, soffset);
        } else {
#pragma unroll
            for (int t = 0; t < L::kKPerWave; ++t) load_to_lds(r, dst_k[t], off_k[t], soffset);
        }
    };
    auto k8_slots = [&](int4v r, int soffset) {
        if constexpr (L::kK8Loads % kWavesPerGroup == 0) {
            load_slots(r, dst_k8[0], off_k8, soffset);
        } else {
#pragma unroll
            for (int t = 0; t < L::kK8PerWave; ++t) load_to_lds(r, dst_k8[t], off_k8[t], soffset);
        }
    };
    // V into buffer `buffer` (0 or 1); spare slots keep their landing area.
    auto v_slots = [&](int4v r, int soffset, int buffer) {
        const unsigned shift = buffer ? static_cast<unsigned>(L::kV1Offset) : 0u;
        if constexpr (L::kVLoads % kWavesPerGroup == 0) {
            load_slots(r, dst_v[0] + shift, off_v, soffset);
        } else {
#pragma unroll
            for (int t = 0; t < L::kVPerWave; ++t)
                load_to_lds(r, dst_v[t] == lds_spare_address ? dst_v[t] : dst_v[t] + shift, off_v[t], soffset);
        }
    };
    // K (FP16 cells) and K8 (INT8 cells) of tile j.
    auto issue_k = [&](int j, bool need16, bool need8) {
        const int k0 = j * kTileKeys;
        if constexpr (kVector) {
            const bool tail = k0 + kTileKeys > N;
            if (need16) {
                if (tail) k_slots(rsrc_from(rsrc_k, k0 * k_row_bytes), 0);
                else k_slots(rsrc_k, k0 * k_row_bytes);
            }
            if (need8) {
                if (tail) k8_slots(rsrc_from(rsrc_k8, k0 * d), 0);
                else k8_slots(rsrc_k8, k0 * d);
            }
        } else {
            if (need16) {
                for (int e = tid; e < kTileKeys * kDP; e += kThreadsPerGroup) {
                    const int row = e / kDP, f = e % kDP, key = k0 + row;
                    *reinterpret_cast<std::uint16_t*>(lds_k + L::k_at(row, 2 * f)) =
                        (key < N && f < d) ? Kh[static_cast<std::int64_t>(key) * p.k_row + f] : 0;
                }
            }
            if (need8) {
                for (int e = tid; e < kTileKeys * L::kDP8; e += kThreadsPerGroup) {
                    const int row = e / L::kDP8, f = e % L::kDP8, key = k0 + row;
                    lds_k8[L::k8_at(row, f)] =
                        (key < N && f < d) ? static_cast<unsigned char>(K8h[static_cast<std::int64_t>(key) * d + f]) : 0;
                }
            }
        }
    };
    auto issue_v = [&](int j, int buffer) {
        const int k0 = j * kTileKeys;
        if constexpr (kVector) {
            if (k0 + kTileKeys > N) v_slots(rsrc_from(rsrc_v, k0 * v_row_bytes), 0, buffer);
            else v_slots(rsrc_v, k0 * v_row_bytes, buffer);
        } else {
            unsigned char* const dst = lds_v + (buffer ? L::kV1Offset : 0);
            for (int e = tid; e < kTileKeys * kDP; e += kThreadsPerGroup) {
                const int row = e / kDP, f = e % kDP, key = k0 + row;
                *reinterpret_cast<std::uint16_t*>(dst + L::v_at(row, 2 * f)) =
                    (key < N && f < d) ? Vh[static_cast<std::int64_t>(key) * p.v_row + f] : 0;
            }
        }
    };
    // Own loads complete (vmcnt 0), then the workgroup barrier.
    auto tile_barrier = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
    };

    // Per-lane LDS offsets of the K fragment (feature chunk dc, key block 0)
    // and V^T fragment (feature block fb, key step 0) reads; key blocks and
    // steps add whole rows (multiples of 16, which keep the chunk rotation).
    // K / K8 fragments: lane (q, h) reads key q of the key block, 16 bytes
    // at feature chunk c. V^T fragments (ds_read_b64_tr_b16): the 16-lane
    // group (fh, h) = ((lane / 16) & 1, lane / 32) reads keys 4h .. 4h + 3
    // (then 8 + 4h ..) x features 16 fb + fh kDP / 2 .. + 15, lane i
    // receiving feature 16 fb + fh kDP / 2 + i (output row 16 fh + i).
    int k_lane[kQC], v_lane[kOB], k8_lane[kQ8C];
#pragma unroll
    for (int m = 0; m < kQ8C; ++m) k8_lane[m] = L::k8_at(q, 32 * m + 16 * h);
#pragma unroll
    for (int c = 0; c < kQC; ++c) k_lane[c] = L::k_at(q, 32 * c + 16 * h);
#pragma unroll
    for (int fb = 0; fb < kOB; ++fb)
        v_lane[fb] = L::v_at(4 * h + (i >> 2), 2 * (16 * fb + (kDP / 2) * ((lane >> 4) & 1) + 4 * (i & 3)));
    // ---------------------------------------------------------- key loop
    RowState<kOB> st;
#pragma unroll
    for (int fb = 0; fb < kOB; ++fb) st.o[fb] = float16v{};
    st.lsum = 0.0f;
    st.m = -INFINITY;
    const bool positive_scale = p.score_scale >= 0.0f;

    const int key_tiles64 = (N - 1) / kTileKeys + 1;
    int tiles = key_tiles64;
    if (p.causal) tiles = min(tiles, (q0 + kRowsPerGroup - 1) / kTileKeys + 1);
    // A split workgroup covers its own range of key tiles.
    const int tile_begin = kSplit ? split * p.split_tiles : 0;
    if constexpr (kSplit) tiles = max(tile_begin, min(tiles, tile_begin + p.split_tiles));
    const std::int64_t trace_base = head * static_cast<std::int64_t>(p.q_tiles16) * p.key_tiles32;
    auto write_trace = [&](int j, std::uint32_t int8_mask, std::uint32_t skip_mask) {
        if (wave == 0 && lane < 16) {
            const int qt = qt0 + (lane >> 1), kt = 2 * j + (lane & 1);
            if (qt < p.q_tiles16 && kt < p.key_tiles32)
                p.trace[trace_base + static_cast<std::int64_t>(qt) * p.key_tiles32 + kt] =
                    static_cast<std::uint8_t>(((skip_mask >> lane) & 1u) ? 2u : ((int8_mask >> lane) & 1u));
        }
    };
    auto needs16 = [](std::uint32_t int8_mask, std::uint32_t skip_mask) {
        return ((~int8_mask & ~skip_mask) & 0xffffu) != 0;
    };

    // The loop visits tiles tile_begin .. tiles - 1 in the order of `step`;
    // in_walk(j) says whether j is still inside that range. The walk starts
    // at one end (tiles >= tile_begin: N >= 1, and a split's range is
    // clamped) and moves by one tile, so it reaches tile_end exactly.
    const int tile_end = step > 0 ? tiles : tile_begin - 1;
    auto in_walk = [&](int j) { return j != tile_end; };
    // Tiles whose 16 cells are all skipped are stepped over: next_tile(j)
    // returns the first tile from j on (in the walk's order) with a visible
    // cell, or the first tile past the range, with that tile's masks,
    // writing the routing trace of the tiles it passes.
    std::uint32_t cur_int8 = 0, cur_skip = 0;
    auto next_tile = [&](int j) {
        for (; in_walk(j); j += step) {
            tile_masks(j, cur_int8, cur_skip);
            if (kDots && p.trace) write_trace(j, cur_int8, cur_skip);
            if (cur_skip != 0xffffu) break;
        }
        return j;
    };
    // Tile j's V sits in buffer v_buffer. The loads of the next visible tile
    // (K, K8, and V into the other buffer) are issued after the tile's second
    // barrier: by then every wave has finished its scores (the K and K8
    // buffers are free) and the previous tile's P.V (its V buffer is free).
    int j = next_tile(step > 0 ? tile_begin : tiles - 1);
    int v_buffer = 0;
    if (in_walk(j)) {
        issue_k(j, needs16(cur_int8, cur_skip), cur_int8 != 0);
        issue_v(j, v_buffer);
    }

    // One iteration per visible tile. A wave with no visible key in the tile
    // (rows above a causal diagonal, or all its cells skipped) takes part in
    // the tile's loads and barriers only: its probabilities would all be 0,
    // so the softmax and P.V would leave m, l and O unchanged.
    while (in_walk(j)) {
        const int k0 = j * kTileKeys;
        const std::uint32_t int8_mask = cur_int8, skip_mask = cur_skip;
        tile_barrier();  // K_j, V_j landed; every wave finished P.V of the previous tile
        set_priority<2>();  // second half of the MFMA phase (P.V, then these scores)

        const unsigned wave_int8 = (int8_mask >> (4 * wave)) & 0xfu;
        const unsigned wave_skip = (skip_mask >> (4 * wave)) & 0xfu;
        const bool active = qw < M && wave_skip != 0xfu && !(p.causal && k0 > qw + kRowsPerWave - 1);
        // Tiles needing no element mask and a non-negative scale use the fast
        // path: raw MFMA results go straight into the exponent FMA.
        const bool masked = k0 + kTileKeys > N || (p.causal && k0 + kTileKeys - 1 > qw);
        const bool fast = positive_scale && !masked;

        float16v s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[kb][e] = -INFINITY;
        float c = 1.0f;
        if (active) {
            float k_factor = 0.0f;  // q_scale * k_scale * score_scale * log2(e)
            if (wave_int8) {
                const float k_scale = half_bits_to_float(load_uniform_u16(p.k_scales + head * p.k_blocks + j));
                k_factor = ((q_scale * k_scale) * p.score_scale) * kLog2e;
            }
            // ---- scores S^T[kb]: lane (q, h) holds row q against keys 32 kb + 8 (e / 4) + 4 h + e % 4
            auto fp16_scores = [&]() {
                // Feature chunk outermost (two independent accumulator
                // chains), K fragments read two chunks ahead.
                s[0] = float16v{};
                s[1] = float16v{};
                half8 kf[3][2];
                auto load_c = [&](int cc, half8 (&dst)[2]) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        dst[kb] = *reinterpret_cast<const half8*>(lds_k + 32 * L::kKStride * kb + k_lane[cc]);
                };
                load_c(0, kf[0]);
                load_c(1, kf[1]);
#pragma unroll
                for (int cc = 0; cc < kQC; ++cc) {
                    if (cc + 2 < kQC) load_c(cc + 2, kf[(cc + 2) % 3]);
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[cc % 3][kb], qf[cc], s[kb], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            // Exact int32 dots of both key blocks.
            auto int8_scores = [&](int16v (&acc)[2]) {
                acc[0] = int16v{};
                acc[1] = int16v{};
                int4v kf8[2][2];
                auto load_m = [&](int m, int4v (&dst)[2]) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        dst[kb] = *reinterpret_cast<const int4v*>(lds_k8 + 32 * L::kK8Stride * kb + k8_lane[m]);
                };
                load_m(0, kf8[0]);
#pragma unroll
                for (int m = 0; m < kQ8C; ++m) {
                    if (m + 1 < kQ8C) load_m(m + 1, kf8[(m + 1) & 1]);
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        acc[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf8[m & 1][kb], q8f[m], acc[kb], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            // Raw int32 dots of key block kb (verification output).
            auto store_dots = [&](int kb, const int16v& acc) {
                const int query = qw + q;
                std::int32_t* row = p.dots + head * static_cast<std::int64_t>(M) * N +
                                    static_cast<std::int64_t>(query) * N;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = k0 + 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (query < M && key < N && !(p.causal && key > query)) row[key] = acc[e];
                }
            };
            const int qh = q >> 4;  // the lane's 16-row routing cell of the wave
            if (wave_skip == 0 && wave_int8 == 0) {
                fp16_scores();
                c = p.score_log2;
            } else if (wave_skip == 0 && wave_int8 == 0xfu) {
                int16v acc[2];
                int8_scores(acc);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    if (kDots && p.dots) store_dots(kb, acc[kb]);
#pragma unroll
                    for (int e = 0; e < 16; ++e) s[kb][e] = static_cast<float>(acc[kb][e]);
                }
                c = k_factor;
            } else {
                // Mixed routes inside the wave: both score kinds where present,
                // explicitly scaled, then selected per lane (cell bit 2 qh + kb).
                const unsigned wave_fp16 = ~(wave_int8 | wave_skip) & 0xfu;
                if (wave_fp16) {
                    fp16_scores();
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) s[kb] *= p.score_log2;
                } else {
                    s[0] = float16v{};
                    s[1] = float16v{};
                }
                if (wave_int8) {
                    int16v acc[2];
                    int8_scores(acc);
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
                        const bool cell_int8 = (wave_int8 >> (2 * qh + kb)) & 1u;
                        if (kDots && p.dots && cell_int8) store_dots(kb, acc[kb]);
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            s[kb][e] = cell_int8 ? static_cast<float>(acc[kb][e]) * k_factor : s[kb][e];
                    }
                }
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    if ((wave_skip >> (2 * qh + kb)) & 1u)
#pragma unroll
                        for (int e = 0; e < 16; ++e) s[kb][e] = -INFINITY;
                c = 1.0f;
            }
            if (!fast && c != 1.0f) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) s[kb] *= c;
                c = 1.0f;
            }
            // ---- element masks: key tail and causal diagonal (explicit scores)
            if (masked) {
                const int query = qw + q;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int key = k0 + 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                        if (key >= N || (p.causal && key > query)) s[kb][e] = -INFINITY;
                    }
            }
        }


        tile_barrier();  // every wave finished reading K_j (and P.V of the previous tile)
        set_priority<0>();  // first half of the VALU phase
        const int j_next = next_tile(j + step);
        if (in_walk(j_next)) {
            issue_k(j_next, needs16(cur_int8, cur_skip), cur_int8 != 0);
            issue_v(j_next, v_buffer ^ 1);
        }

        // ---- online softmax, then O^T += V^T P^T
        if (active) {
            half8 ph[4], pl[4];
            softmax_tile<kOB, kPrecise>(st, s, c, ph, pl);
            {
                // V^T fragment of step t = (key step t / kOB, feature block
                // t % kOB), read kAhead steps before its MFMA.
                auto v_frag = [&](int t) {
                    const unsigned char* v_lo = lds_v + (v_buffer ? L::kV1Offset : 0) + 16 * L::kVStride * (t / kOB) + v_lane[t % kOB];
                    return concat(read_tr16(v_lo), read_tr16(v_lo + 8 * L::kVStride));
                };
                constexpr int kSteps = 4 * kOB;
                constexpr int kAhead = 3;
                set_priority<0>();  // first half of the MFMA phase
                half8 vf[kAhead + 1];
#pragma unroll
                for (int t = 0; t < kAhead; ++t)
                    if (t < kSteps) vf[t] = v_frag(t);
#pragma unroll
                for (int t = 0; t < kSteps; ++t) {
                    if (t + kAhead < kSteps) vf[(t + kAhead) % (kAhead + 1)] = v_frag(t + kAhead);
                    const int ks = t / kOB, fb = t % kOB;
                    st.o[fb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[t % (kAhead + 1)], ph[ks], st.o[fb], 0, 0, 0);
                    if constexpr (kPrecise)
                        st.o[fb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[t % (kAhead + 1)], pl[ks], st.o[fb], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        j = j_next;
        v_buffer ^= 1;
    }

    // Routing trace of tiles a causal workgroup never visits.
    if (kDots && !kSplit && p.trace && tiles < key_tiles64) {
        for (int j = tiles; j < key_tiles64; ++j) {
            std::uint32_t int8_mask = 0, skip_mask = 0;
            tile_masks(j, int8_mask, skip_mask);
            write_trace(j, int8_mask, skip_mask);
        }
    }

    // fp32 rows of 128 or 64 features (O, or a split's partial rows) leave
    // the variants without dot export through LDS. From registers, each
    // store instruction writes 16 bytes to each of 32 rows, i.e. 32 partial
    // cache lines, and those lines, held in the XCD's L2 until written back,
    // evict K / V tiles. Staged, each store writes 8 rows x 128 bytes (full
    // cache lines) with a non-temporal hint, so the rows bypass the L2. The stage buffers
    // are the K tile buffer (both 4 KiB regions of it at d = 64, all four
    // at d = 128) and at d = 64 the V buffer the last tile did not use:
    // every wave has passed the last tile's second barrier, so no wave
    // reads them any more and no load targets them. Each wave stages its
    // 32 rows in kDP / 32 passes of 32 features through a 4 KiB region.
    // out / out_row: the head's first row and the distance between rows, in
    // floats; every value is multiplied by factor.
    constexpr bool kStaged = kVector && !kDots && (kDP == 128 || kDP == 64);
    auto store_staged = [&](float* out, std::int64_t out_row, float factor) {
        if constexpr (kStaged) {
            constexpr int kRowBytes = 128;           // 32 features per pass
            constexpr int kRegion = 32 * kRowBytes;  // 4 KiB per wave
            constexpr int kPasses = kDP / 32;
            constexpr int kPassesPerHalf = kPasses / 2;  // passes over features [0, kDP / 2)
            unsigned char* region;
            if constexpr (kDP == 128) {
                static_assert(L::kKBytes >= kWavesPerGroup * kRegion, "stage regions fit the K buffer");
                region = lds_k + wave * kRegion;
            } else {
                static_assert(L::kKBytes >= 2 * kRegion && L::kVBytes >= 2 * kRegion, "stage regions fit K and V");
                region = wave < 2 ? lds_k + wave * kRegion : lds_v + (v_buffer ? L::kV1Offset : 0) + (wave - 2) * kRegion;
            }
            // The lane's position, taken afresh here: the stage addresses
            // depend on the lane only, and computed before the key loop
            // they would hold registers through it.
            int me = lane;
            asm volatile("" : "+v"(me));
            const int my_q = me & 31, my_h = me >> 5;
            const int c = me & 7, sub = me >> 3;  // read side: chunk c of row sub of each 8-row piece
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                // Features 32 pass .. 32 pass + 31: slots
                // r4 = 2 (pass / kPassesPerHalf) + r of blocks
                // fb = 2 (pass % kPassesPerHalf) + b hold features
                // 32 pass + 16 b + 8 r + 4 h (+ 0..3) of row q, i.e. 16-byte
                // chunk 4 b + 2 r + h of the pass, stored rotated by the row.
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const int r4 = 2 * (pass / kPassesPerHalf) + r, fb = 2 * (pass % kPassesPerHalf) + b;
                        const float4v value{st.o[fb][4 * r4], st.o[fb][4 * r4 + 1], st.o[fb][4 * r4 + 2],
                                            st.o[fb][4 * r4 + 3]};
                        const int chunk = 4 * b + 2 * r + my_h;
                        *reinterpret_cast<float4v*>(region + my_q * kRowBytes + (((chunk + my_q) & 7) << 4)) =
                            value * factor;
                    }
                // Piece i: rows 8 i .. 8 i + 7 of the wave, 8 lanes per row.
                // Every read is issued before any store (the reads stay in
                // the wave's region; only the stores depend on the row).
                float4v piece[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int local = 8 * i + sub;
                    piece[i] = *reinterpret_cast<const float4v*>(region + local * kRowBytes + (((c + local) & 7) << 4));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(piece[i]));  // keep the reads here
                float* const first = out + static_cast<std::int64_t>(qw + sub) * out_row + 32 * pass + 4 * c;
                const std::int64_t piece_step = 8 * out_row;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (qw + 8 * i + sub < M)
                        __builtin_nontemporal_store(piece[i], reinterpret_cast<float4v*>(first + i * piece_step));
            }
        }
    };
    // ---------------------------------------------------------- epilogue
    if constexpr (kSplit) {
        // This split's unnormalised rows and their (m, l), for the combine.
        float a = st.lsum, b = st.lsum;
        permlane32_swap(a, b);
        const int row = qw + q;
        if constexpr (kStaged) {
            if (d == kDP) {
                store_staged(p.part_o + static_cast<std::int64_t>(split) * M * d, d, 1.0f);
                if (row < M && h == 0) {
                    float* const ml = p.part_ml + 2 * (static_cast<std::int64_t>(split) * M + row);
                    ml[0] = st.m;
                    ml[1] = a + b;
                }
                return;
            }
        }
        if (row < M) {
            unsigned char* const part = reinterpret_cast<unsigned char*>(p.part_o + static_cast<std::int64_t>(split) * M * d);
            const std::int64_t row_offset = static_cast<std::int64_t>(row) * d;
#pragma unroll
            for (int fb = 0; fb < kOB; ++fb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int feature = (r4 < 2 ? 0 : kDP / 2 - 16) + 16 * fb + 8 * r4 + 4 * h;
                    const float4v value{st.o[fb][4 * r4], st.o[fb][4 * r4 + 1], st.o[fb][4 * r4 + 2], st.o[fb][4 * r4 + 3]};
                    store_output(part, TILEMIX_DTYPE_F32, row_offset + feature, value, d - feature, kVector);
                }
            if (h == 0) {
                float* const ml = p.part_ml + 2 * (static_cast<std::int64_t>(split) * M + row);
                ml[0] = st.m;
                ml[1] = a + b;
            }
        }
    } else {
        float a = st.lsum, b = st.lsum;
        permlane32_swap(a, b);  // the row's other half, held by lane ^ 32
        const float l = a + b;
        const float inverse = l > 0.0f ? 1.0f / l : 0.0f;
        const int row = qw + q;
        if constexpr (kStaged) {
            if (p.o_dtype == TILEMIX_DTYPE_F32 && d == kDP) {
                store_staged(reinterpret_cast<float*>(Oh), p.o_row, inverse);
                return;
            }
        }
        if (row < M) {
            const std::int64_t row_offset = static_cast<std::int64_t>(row) * p.o_row;
#pragma unroll
            for (int fb = 0; fb < kOB; ++fb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    // Output row R = 8 r4 + 4 h (+ 0..3) of block fb is feature
                    // 16 fb + R (R < 16) or kDP / 2 + 16 fb + R - 16.
                    const int feature = (r4 < 2 ? 0 : kDP / 2 - 16) + 16 * fb + 8 * r4 + 4 * h;
                    const float4v value{st.o[fb][4 * r4], st.o[fb][4 * r4 + 1], st.o[fb][4 * r4 + 2], st.o[fb][4 * r4 + 3]};
                    store_output(Oh, p.o_dtype, row_offset + feature, value * inverse, d - feature, kVector);
                }
        }
    }
}

// O of a key-range split launch: per row, m = max over the splits of m_s,
// O = sum_s 2^(m_s - m) O_s / sum_s 2^(m_s - m) l_s (log2-domain row states;
// splits whose rows saw no key have m_s = -inf and weigh nothing). One
// thread per row and 4 features, splits summed in order. Splits are taken
// kBatch at a time, every load of a batch issued before any use (one memory
// round trip per batch); m is the maximum over the splits seen so far, and a
// later batch that raises it rescales the sums (up to kBatch splits: one
// batch, m over all splits).
template <bool kVector>
__global__ __launch_bounds__(256) void split_combine_kernel(const float* part_o, const float* part_ml, int splits,
                                                           int M, int d, float* O, std::int64_t o_row) {
    constexpr int kBatch = 16;
    const int groups = (d + 3) / 4;
    const std::int64_t index = static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (index >= static_cast<std::int64_t>(M) * groups) return;
    const int row = static_cast<int>(index / groups);
    const int f0 = 4 * static_cast<int>(index - static_cast<std::int64_t>(row) * groups);
    const float2v* const ml = reinterpret_cast<const float2v*>(part_ml);
    float m = -INFINITY, l = 0.0f;
    float4v acc{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < splits; s0 += kBatch) {
        float2v state[kBatch];
        float4v value[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const std::int64_t r = static_cast<std::int64_t>(s0 + b < splits ? s0 + b : s0) * M + row;
            state[b] = ml[r];
            const float* src = part_o + r * d + f0;
            if constexpr (kVector) {
                value[b] = *reinterpret_cast<const float4v*>(src);
            } else {
                for (int e = 0; e < 4; ++e) value[b][e] = f0 + e < d ? src[e] : 0.0f;
            }
        }
        float m_next = m;
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (s0 + b < splits) m_next = fmaxf(m_next, state[b][0]);
        if (m_next == -INFINITY) continue;  // no split so far saw a key of this row
        if (m_next != m) {
            const float rescale = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_next);
            l *= rescale;
            acc *= rescale;
            m = m_next;
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const float w = (s0 + b >= splits || state[b][0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(state[b][0] - m);
            l += w * state[b][1];
            acc += w * value[b];
        }
    }
    const float inverse = l > 0.0f ? 1.0f / l : 0.0f;
    float* dst = O + static_cast<std::int64_t>(row) * o_row + f0;
    if constexpr (kVector) {
        *reinterpret_cast<float4v*>(dst) = acc * inverse;
    } else {
        for (int e = 0; e < 4 && f0 + e < d; ++e) dst[e] = acc[e] * inverse;
    }
}

template <int DC, bool kVector, bool kPrecise, bool kDots, bool kSplit>
hipError_t launch_variant(const AttnParams& p, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(p.q_blocks) * static_cast<unsigned>(p.heads) *
                            static_cast<unsigned>(kSplit ? p.splits : 1);
    attention_kernel<DC, kVector, kPrecise, kDots, kSplit><<<blocks, kThreadsPerGroup, 0, stream>>>(p);
    return hipGetLastError();
}

// Split launches exist for the per-head entry point only, whose P.V is
// always the precise one.
template <int DC, bool kVector>
hipError_t launch_vp(const AttnParams& p, bool precise, bool dots, hipStream_t stream) {
    if (p.splits > 1) {
        if (!precise) return hipErrorInvalidValue;
        return dots ? launch_variant<DC, kVector, true, true, true>(p, stream)
                    : launch_variant<DC, kVector, true, false, true>(p, stream);
    }
    if (precise)
        return dots ? launch_variant<DC, kVector, true, true, false>(p, stream)
                    : launch_variant<DC, kVector, true, false, false>(p, stream);
    return dots ? launch_variant<DC, kVector, false, true, false>(p, stream)
                : launch_variant<DC, kVector, false, false, false>(p, stream);
}

template <int DC>
hipError_t launch_dc(const AttnParams& p, bool vector, bool precise, hipStream_t stream) {
    const bool dots = p.dots != nullptr || p.trace != nullptr;
    return vector ? launch_vp<DC, true>(p, precise, dots, stream) : launch_vp<DC, false>(p, precise, dots, stream);
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
// on every call, src/tilemix.cu:254-260), with the device's compute-unit
// count (0 when the device is not cached).
constexpr int kMaxDevices = 64;

hipError_t check_device(int* compute_units = nullptr) {
    static std::atomic<int> verdict[kMaxDevices];  // 0 unknown, 1 supported, 2 unsupported
    static std::atomic<int> units[kMaxDevices];
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return status;
    const bool cached = device >= 0 && device < kMaxDevices;
    if (compute_units) *compute_units = 0;
    if (cached) {
        const int known = verdict[device].load(std::memory_order_relaxed);
        if (known == 2) return hipErrorNotSupported;
        if (known == 1) {
            if (compute_units) *compute_units = units[device].load(std::memory_order_relaxed);
            return hipSuccess;
        }
    }
    hipDeviceProp_t properties{};
    status = hipGetDeviceProperties(&properties, device);
    if (status != hipSuccess) return status;
    const bool supported = std::strncmp(properties.gcnArchName, "gfx950", 6) == 0;
    if (cached) {
        units[device].store(properties.multiProcessorCount, std::memory_order_relaxed);
        verdict[device].store(supported ? 1 : 2, std::memory_order_relaxed);
        if (compute_units) *compute_units = properties.multiProcessorCount;
    }
    return supported ? hipSuccess : hipErrorNotSupported;
}

hipError_t launch_attention(AttnParams p, bool precise, hipStream_t stream) {
    if (static_cast<long long>(p.q_blocks) * p.heads > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    int units = 0;
    hipError_t status = check_device(&units);
    if (status != hipSuccess) return status;
    // Non-causal heads in the per-XCD head-major order whose query blocks
    // outnumber an XCD's workgroup slots stream K / V once per round of
    // slots; alternate rounds walk the keys in opposite directions.
    const int xcd_slots = units / kXcds * kGroupsPerCU;
    p.reverse_slots = (!p.causal && p.splits <= 1 && p.heads % kXcds == 0 && xcd_slots > 0 && p.q_blocks > xcd_slots)
                          ? xcd_slots : 0;
    // The vector path moves 16-byte pieces and addresses a head's K / V with
    // 32-bit buffer offsets; other shapes take the element-wise path.
    const std::int64_t k_range = (static_cast<std::int64_t>(p.N - 1) * p.k_row + p.d) * 2;
    const std::int64_t v_range = (static_cast<std::int64_t>(p.N - 1) * p.v_row + p.d) * 2;
    bool vector = p.d % 16 == 0 && aligned(p.Q, 16) && aligned(p.K, 16) && aligned(p.V, 16) &&
                  aligned(p.O, 16) && p.q_stride % 8 == 0 && p.k_stride % 8 == 0 &&
                  p.v_stride % 8 == 0 && p.o_stride % 4 == 0 && p.q_row % 8 == 0 &&
                  p.k_row % 8 == 0 && p.v_row % 8 == 0 && p.o_row % 4 == 0 &&
                  k_range < (std::int64_t{1} << 31) && v_range < (std::int64_t{1} << 31);
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

}  // namespace
}  // namespace tilemix

// Workspace of the per-head entry point's key-range split (partial O rows and
// row states of every split, [splits][M][d] + [splits][M][2] fp32). One copy
// per GPU, held until the process ends; the library allocates nothing.
// Split calls on a device are ordered through one event (each waits for the
// previous split call's combine, whatever its stream), so concurrent streams
// never share it at once; calls made while their stream is being captured
// into a graph take the plain launch instead.
static constexpr std::size_t kSplitScratchFloats = std::size_t{8} << 20;  // 32 MiB
static __device__ __align__(256) float split_scratch[kSplitScratchFloats];

namespace tilemix {
namespace {

// A split covers at least this many key tiles, and a head with fewer than
// kMinSplitHead key tiles is not split: the split's fixed cost (partial rows,
// the combine launch, the ordering event) is about that of a few tiles'
// walk. Measured per call (M = 4096, d = 128): at N = 256 the plain launch
// is 23 % faster than two splits; at N = 512 four 2-tile splits are 14 %
// faster than two 4-tile ones, and the reference demo (16 tiles) 7 % with 8
// splits than with 4; from N = 4096 on the slot count limits the splits.
constexpr int kMinSplitTiles = 2;
constexpr int kMinSplitHead = 8;

struct SplitDevice {
    float* scratch = nullptr;
    hipEvent_t done = nullptr;
    bool recorded = false;
};

std::mutex& split_lock() {
    static std::mutex lock;
    return lock;
}

SplitDevice* split_devices() {
    static SplitDevice devices[kMaxDevices];
    return devices;
}

// Key-range splits for a single-head, non-causal launch of at least
// kMinSplitHead key tiles that would fill less than half of the device's
// workgroup slots: as many as bring it to one wave of workgroups, each
// covering at least kMinSplitTiles key tiles and all fitting in the
// workspace (1 = no split).
int choose_splits(const AttnParams& p, int compute_units) {
    if (compute_units <= 0 || p.heads != 1 || p.causal) return 1;
    const int resident = compute_units * kGroupsPerCU;
    if (2 * p.q_blocks > resident) return 1;
    const int tiles = (p.N - 1) / kTileKeys + 1;
    if (tiles < kMinSplitHead) return 1;
    int splits = std::min(resident / p.q_blocks, tiles / kMinSplitTiles);
    while (splits > 1 && static_cast<std::size_t>(splits) * p.M * (p.d + 2) > kSplitScratchFloats) --splits;
    return splits > 1 ? splits : 1;
}

// launch_attention, with the key range split over several workgroups per
// 128-row block when choose_splits says so: the attention kernel writes each
// split's partial rows to the workspace, split_combine_kernel merges them
// into O, both on `stream`.
hipError_t launch_attention_split(AttnParams p, bool precise, hipStream_t stream) {
    int units = 0;
    hipError_t status = check_device(&units);
    if (status != hipSuccess) return status;
    int splits = choose_splits(p, units);
    if (splits > 1) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) splits = 1;
    }
    int device = 0;
    if (splits > 1 && (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)) splits = 1;
    if (splits <= 1) return launch_attention(p, precise, stream);

    std::lock_guard<std::mutex> guard(split_lock());
    SplitDevice& state = split_devices()[device];
    if (!state.scratch || !state.done) {
        // First split call on this device: another thread may be capturing a
        // graph in global mode, which would reject these runtime calls (they
        // enqueue no work), so this thread's capture mode is relaxed around
        // them and then restored.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        status = hipThreadExchangeStreamCaptureMode(&mode);
        if (status != hipSuccess) return status;
        if (!state.scratch) {
            void* address = nullptr;
            status = hipGetSymbolAddress(&address, HIP_SYMBOL(split_scratch));
            if (status == hipSuccess) state.scratch = static_cast<float*>(address);
        }
        if (status == hipSuccess && !state.done) status = hipEventCreateWithFlags(&state.done, hipEventDisableTiming);
        const hipError_t restored = hipThreadExchangeStreamCaptureMode(&mode);
        if (status != hipSuccess) return status;
        if (restored != hipSuccess) return restored;
    }
    if (state.recorded) {
        status = hipStreamWaitEvent(stream, state.done, 0);
        if (status != hipSuccess) return status;
    }
    const int tiles = (p.N - 1) / kTileKeys + 1;
    p.split_tiles = (tiles + splits - 1) / splits;
    p.splits = (tiles + p.split_tiles - 1) / p.split_tiles;
    p.part_o = state.scratch;
    p.part_ml = state.scratch + static_cast<std::size_t>(p.splits) * p.M * p.d;
    status = launch_attention(p, precise, stream);
    if (status != hipSuccess) return status;
    float* const O = static_cast<float*>(p.O);
    const std::int64_t threads = static_cast<std::int64_t>(p.M) * ((p.d + 3) / 4);
    const unsigned blocks = static_cast<unsigned>((threads + 255) / 256);
    if (p.d % 4 == 0 && aligned(O, 16) && p.o_row % 4 == 0)
        split_combine_kernel<true><<<blocks, 256, 0, stream>>>(p.part_o, p.part_ml, p.splits, p.M, p.d, O, p.o_row);
    else
        split_combine_kernel<false><<<blocks, 256, 0, stream>>>(p.part_o, p.part_ml, p.splits, p.M, p.d, O, p.o_row);
    status = hipGetLastError();
    if (status != hipSuccess) return status;
    status = hipEventRecord(state.done, stream);
    if (status != hipSuccess) return status;
    state.recorded = true;
    return hipSuccess;
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
    p.group_shift = (group & (group - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(group)) : -1;
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
    p.q_row = p.k_row = p.v_row = p.o_row = d;
    p.o_dtype = TILEMIX_DTYPE_F32;
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
    // A head too small to fill the device has its key range split.
    return launch_attention_split(p, /*precise=*/true, static_cast<hipStream_t>(stream));
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
    if (a.o_dtype < TILEMIX_DTYPE_F32 || a.o_dtype > TILEMIX_DTYPE_BF16) return hipErrorInvalidValue;
    const std::int64_t q_row = a.q_row_stride ? a.q_row_stride : a.d;
    const std::int64_t k_row = a.k_row_stride ? a.k_row_stride : a.d;
    const std::int64_t v_row = a.v_row_stride ? a.v_row_stride : a.d;
    const std::int64_t o_row = a.o_row_stride ? a.o_row_stride : a.d;
    if (!strided_heads_ok(a.heads, a.M, a.d, a.q_head_stride, q_row) ||
        !strided_heads_ok(a.heads, a.M, a.d, a.o_head_stride, o_row) ||
        !strided_heads_ok(a.heads, a.N, a.d, a.k_head_stride, k_row) ||
        !strided_heads_ok(a.heads, a.N, a.d, a.v_head_stride, v_row))
        return hipErrorInvalidValue;
    const bool int8 = a.route_words != nullptr;
    if (a.quantize < 0 || a.quantize > 2) return hipErrorInvalidValue;
    if (int8) {
        if (!a.K8 || !a.k_scales) return hipErrorInvalidValue;
        if (!a.quantize && (!a.Q8 || !a.q_scales)) return hipErrorInvalidValue;
        if (a.quantize && (!a.Q8) != (!a.q_scales)) return hipErrorInvalidValue;
    } else if (a.score_dots) {
        return hipErrorInvalidValue;
    }
    // Every check precedes the first launch: an error return leaves all
    // outputs (K8 / k_scales of the pre-pass included) untouched.
    if (static_cast<long long>((a.M - 1) / kQBlockRows + 1) * a.heads > 0x7fffffffLL)
        return hipErrorInvalidConfiguration;
    if (a.quantize == 1 && int8) {
        const QuantSide none = make_quant_side(nullptr, nullptr, nullptr, 0, 1, kQBlockRows, a.d);
        const QuantSide k = make_quant_side(a.K, a.K8, a.k_scales, a.k_head_stride, a.N, kKBlockRows, k_row);
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
    p.q_row = q_row;
    p.k_row = k_row;
    p.v_row = v_row;
    p.o_row = o_row;
    p.o_dtype = a.o_dtype;
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
