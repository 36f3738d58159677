#ifndef TILEMIX_CAPI_H
#define TILEMIX_CAPI_H
/*
 * C ABI of the MI355X TileMix library (libtilemix_hip.so).
 *
 * Plain pointers, sizes and ints only, so that ctypes / cgo / JNI / N-API can
 * bind it without C++ or HIP headers:
 *   - fp16 tensors are passed as `uint16_t*` holding IEEE binary16 bit
 *     patterns (the storage of `__half`);
 *   - every pointer is a device pointer owned by the caller; the library
 *     allocates no device memory and keeps no state between calls besides
 *     a cached per-device capability check, the fixed scratch array of
 *     tilemix_tiles_importance_noalloc, and the fixed split workspace and
 *     one ordering event per device of tilemix_attention (see there);
 *   - `stream` is a `hipStream_t` (NULL = the default stream); all work is
 *     enqueued on it and nothing synchronises;
 *   - the return value is a `hipError_t` code (0 = hipSuccess). Argument
 *     errors are reported before any HIP runtime call, so they can be tested
 *     on a machine without a GPU.
 *
 * include/attention_fused.h wraps these in the reference's C++ signatures.
 */
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes returned (numeric values of hipError_t). */
#define TILEMIX_SUCCESS 0                     /* hipSuccess */
#define TILEMIX_ERROR_INVALID_VALUE 1         /* hipErrorInvalidValue */
#define TILEMIX_ERROR_INVALID_CONFIGURATION 9 /* hipErrorInvalidConfiguration */
#define TILEMIX_ERROR_NOT_SUPPORTED 801       /* hipErrorNotSupported */

/*
 * Replaces quantize_tilemix_qk (reference include/attention_fused.h:62-65,
 * src/tilemix.cu:223-236).
 * Symmetric INT8 quantization of Q in 128-row blocks and K in 64-row blocks:
 * scale = fp32(absmax / 127) (IEEE round-to-nearest), stored as fp16;
 * value = clamp(trunc(x/scale + copysign(0.5, x/scale)), -127, 127), 0 when
 * the block is all zeros. Q8[M*d], K8[N*d], q_scales[ceil(M/128)],
 * k_scales[ceil(N/64)]. Errors: null pointer or M, N, d <= 0 ->
 * InvalidValue; d > 128 -> NotSupported.
 */
int tilemix_quantize_qk(const uint16_t* Q, const uint16_t* K, int8_t* Q8, int8_t* K8,
                        uint16_t* q_scales, uint16_t* k_scales, int M, int N, int d,
                        void* stream);

/*
 * Replaces launch_fused_fp16_attention (reference include/attention_fused.h:68-72,
 * src/tilemix.cu:238-278); TileMixRouting and TileMixQuantized
 * (attention_fused.h:47-60) are flattened into their fields.
 * O[M*d] (fp32) = softmax(score_scale * route(Q K^T)) V for one head, where
 * the route of each 16-row x 32-key cell is bit (ktile / key_tiles_per_group)
 * of routing word [qtile * words_per_row + group / 64]: 1 = INT8 scores
 * (exact int32 dot of Q8/K8 rows times q_scales[q/128] * k_scales[k/64]),
 * 0 = FP16 scores (fp16 products, fp32 accumulation). route_words == NULL
 * means every cell is FP16. decoded_bits (optional, ceil(M/16)*ceil(N/32)
 * bytes) receives the decoded bit of every cell; score_dots (optional, M*N
 * int32) receives the raw int32 dot of every INT8-routed (q, k).
 * Validation order and codes follow src/tilemix.cu:242-266.
 * A head too small to fill the device (its 128-row blocks under half of the
 * workgroup slots) with at least 8 key tiles of 64 has its key range split
 * over several workgroups per block, whose partial rows go to a fixed 32 MiB
 * device array inside the library (one per GPU) and are merged into O by a
 * second kernel on `stream`. Split calls on one device are ordered through one event (each
 * waits for the previous one's merge, on any stream); a call made while
 * `stream` is being captured into a graph takes the unsplit launch.
 */
int tilemix_attention(const uint16_t* Q, const uint16_t* K, const uint16_t* V, float* O,
                      int M, int N, int d, float score_scale, void* stream,
                      const uint64_t* route_words, size_t route_word_count,
                      int key_tiles_per_group, uint8_t* decoded_bits,
                      const int8_t* Q8, const int8_t* K8, const uint16_t* q_scales,
                      const uint16_t* k_scales, int32_t* score_dots);

/* Element types of O for the batched entry point (o_dtype). */
#define TILEMIX_DTYPE_F32 0
#define TILEMIX_DTYPE_F16 1
#define TILEMIX_DTYPE_BF16 2

/* Routing codes written to decoded_bits by the batched entry point. */
#define TILEMIX_ROUTE_FP16 0
#define TILEMIX_ROUTE_INT8 1
#define TILEMIX_ROUTE_SKIP 2

/*
 * Batched multi-head problem for tilemix_attention_batched /
 * tilemix_quantize_qk_batched. No reference counterpart: the reference API is
 * one head per call; this runs `heads` independent heads in one launch, each
 * laid out exactly as the per-head API expects (rows of d contiguous
 * elements), head h starting at base + h * <x>_head_stride elements.
 *
 * Extensions over the per-head API:
 *   causal      key k is visible to query q only when k <= q;
 *   skip_words  same packing and size as route_words; a set bit removes the
 *               whole cell (its scores are -inf). A query row left with no
 *               visible key gets O = 0;
 *   precise     0: P is rounded to fp16 for the P.V MFMA (fast);
 *               1: P is split into fp16 hi + lo parts (two MFMAs), giving
 *                  fp32-level accuracy;
 *   quantize    1: the call quantizes Q and K itself: the K blocks are
 *               quantized by a pre-pass into K8 / k_scales (required outputs),
 *               each workgroup quantizes its own 128-row Q block in registers,
 *               and Q8 / q_scales, if non-NULL, receive the Q result;
 *               2: as 1, but K8 / k_scales are caller-provided inputs (e.g.
 *               a key cache quantized once by tilemix_quantize_qk_batched);
 *               0: Q8/K8/q_scales/k_scales are caller-provided inputs (as
 *               produced by tilemix_quantize_qk_batched).
 *               Only INT8-routed cells read the quantized operands, so they
 *               are required only when route_words is non-NULL.
 * Per-head sizes: route/skip words tilemix_routing_word_count(M, N, g);
 * decoded_bits ceil(M/16)*ceil(N/32) bytes; score_dots M*N; Q8 M*d; K8 N*d;
 * q_scales ceil(M/128); k_scales ceil(N/64) - all contiguous per head.
 *
 * Layout and output options (appended; zero keeps the behaviour above):
 *   o_dtype       TILEMIX_DTYPE_F32 (O is float), _F16 or _BF16 (O holds
 *                 16-bit values rounded to nearest even from the same fp32
 *                 result); o_head_stride then counts 16-bit elements;
 *   *_row_stride  elements between consecutive rows of one head (0 = d), so
 *                 e.g. a [B, S, H, D] tensor is head stride D, row stride
 *                 H * D. Heads must not overlap: either each head ends
 *                 before the next begins, or all heads interleave inside
 *                 every row. Q8/K8 stay contiguous [rows][d] per head.
 */
typedef struct TileMixBatchedArgs {
    const uint16_t* Q;
    const uint16_t* K;
    const uint16_t* V;
    float* O;
    int heads;
    int M;
    int N;
    int d;
    int64_t q_head_stride;
    int64_t k_head_stride;
    int64_t v_head_stride;
    int64_t o_head_stride;
    float score_scale;
    int causal;
    int precise;
    int quantize;
    const uint64_t* route_words;
    const uint64_t* skip_words;
    int key_tiles_per_group;
    uint8_t* decoded_bits;
    int8_t* Q8;
    int8_t* K8;
    uint16_t* q_scales;
    uint16_t* k_scales;
    int32_t* score_dots;
    int o_dtype;
    int64_t q_row_stride;
    int64_t k_row_stride;
    int64_t v_row_stride;
    int64_t o_row_stride;
} TileMixBatchedArgs;

/* Multi-head attention (extension, see TileMixBatchedArgs). */
int tilemix_attention_batched(const TileMixBatchedArgs* args, void* stream);

/* Multi-head quantizer (extension): tilemix_quantize_qk for each of `heads`
 * heads, head h of Q/K at h * {q,k}_head_stride elements, outputs contiguous
 * per head (Q8 M*d, K8 N*d, q_scales ceil(M/128), k_scales ceil(N/64)). Either
 * side may be skipped by passing NULL for both its input and outputs. */
int tilemix_quantize_qk_batched(const uint16_t* Q, const uint16_t* K, int8_t* Q8, int8_t* K8,
                                uint16_t* q_scales, uint16_t* k_scales, int heads, int M,
                                int N, int d, int64_t q_head_stride, int64_t k_head_stride,
                                void* stream);

/*
 * Device-side routing-mask producer (no reference counterpart: the reference
 * builds masks on the host, src/tests/tilemix_test.cu:432-448 and
 * src/main.cu:48; this produces the same TileMixRouting word format,
 * include/attention_fused.h:34-52, on the GPU).
 *
 * Tile codes are uint8 [heads][tiles_q][tiles_k] with tiles_q =
 * ceil(M / tile_rows), tiles_k = ceil(N / tile_keys), values
 * TILEMIX_ROUTE_FP16 / _INT8 / _SKIP; tiles must be whole 16-row x 32-key
 * routing cells (tile_rows % 16 == 0, tile_keys % 32 == 0). Random builders
 * draw u = (splitmix64(seed ^ splitmix64(2 * index + salt)) >> 40) / 2^24 for
 * tile linear index (head * tiles_q + i) * tiles_k + j (salt 0), so the codes
 * depend only on (seed, head, tile). Errors: null pointer, non-positive size,
 * bad tile shape or probability outside [0, 1] -> InvalidValue.
 */

/* Packs tile codes into route_words and skip_words, each heads *
 * tilemix_routing_word_count_c(M, N, key_tiles_per_group) words, contiguous
 * per head: bit = INT8 (route) or skip (skip), other codes FP16. A key-tile
 * group must not straddle two tiles: (tile_keys / 32) % key_tiles_per_group
 * == 0, else InvalidValue. */
int tilemix_routes_from_tiles(const uint8_t* tile_codes, int heads, int M, int N, int tile_rows,
                              int tile_keys, int key_tiles_per_group, uint64_t* route_words,
                              uint64_t* skip_words, void* stream);

/* Each tile INT8 when u < p_int8, else FP16. */
int tilemix_tiles_bernoulli(uint8_t* tile_codes, int heads, int M, int N, int tile_rows, int tile_keys,
                            float p_int8, uint64_t seed, void* stream);

/* Square causal problem (M = N = S): tile (i, j) is SKIP
 * when j > last = (i * tile_rows + tile_rows - 1) / tile_keys, FP16 when
 * last - j < fp16_band, otherwise INT8 when u < p_int8, else FP16. */
int tilemix_tiles_causal_band(uint8_t* tile_codes, int heads, int S, int tile_rows, int tile_keys,
                              int fp16_band, float p_int8, uint64_t seed, void* stream);

/* SKIP when u < p_skip, INT8 when u < p_skip + p_int8, else FP16 (BASELINE
 * config 5); a tile row left all SKIP gets tile j = splitmix64(seed ^
 * splitmix64(2 * (head * tiles_q + i) + 1)) % tiles_k forced FP16.
 * p_skip + p_int8 > 1 -> InvalidValue. */
int tilemix_tiles_three_way(uint8_t* tile_codes, int heads, int M, int N, int tile_rows, int tile_keys,
                            float p_skip, float p_int8, uint64_t seed, void* stream);

/* Importance router: per head, the round-half-even(
 * fp16_fraction * tiles_q * tiles_k) tiles with the largest bound
 * d * amax|Q tile rows| * amax|K tile keys| are FP16 (ties to the lower
 * linear tile index), the rest INT8. Head h of Q/K starts at h *
 * {q,k}_head_stride elements (ignored when heads == 1). `workspace` is device
 * scratch of at least tilemix_importance_workspace_bytes(...) bytes (the
 * per-tile maxima); tiles_q + tiles_k > 16384 -> NotSupported. */
size_t tilemix_importance_workspace_bytes(int heads, int M, int N, int tile_rows, int tile_keys);
int tilemix_tiles_importance(const uint16_t* Q, const uint16_t* K, int heads, int M, int N, int d,
                             int64_t q_head_stride, int64_t k_head_stride, int tile_rows, int tile_keys,
                             float fp16_fraction, float* workspace, size_t workspace_bytes,
                             uint8_t* tile_codes, void* stream);

/* tilemix_tiles_importance without a workspace argument: no reference
 * counterpart. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the per-tile maxima live in a fixed scratch array inside the library, one
 * copy per GPU (tilemix_importance_noalloc_max_bytes(), 1 MiB), located once
 * per device with hipGetSymbolAddress on the first call there; the call
 * allocates nothing. Problems needing more than that
 * (tilemix_importance_workspace_bytes(...) > the maximum) -> InvalidValue;
 * other errors as tilemix_tiles_importance. Every call on one GPU shares the
 * scratch, so calls that overlap on one GPU (different streams, threads)
 * race; calls ordered on one stream do not. */
size_t tilemix_importance_noalloc_max_bytes(void);
int tilemix_tiles_importance_noalloc(const uint16_t* Q, const uint16_t* K, int heads, int M, int N, int d,
                                     int64_t q_head_stride, int64_t k_head_stride, int tile_rows, int tile_keys,
                                     float fp16_fraction, uint8_t* tile_codes, void* stream);

/* tilemix_quantize_qk_batched with row strides (elements between consecutive
 * rows of a head, 0 = d) for row-strided Q/K such as [B, S, H, D] tensors;
 * the outputs stay contiguous per head. Head/row strides must not make heads
 * overlap (see TileMixBatchedArgs). */
int tilemix_quantize_qk_strided(const uint16_t* Q, const uint16_t* K, int8_t* Q8, int8_t* K8,
                                uint16_t* q_scales, uint16_t* k_scales, int heads, int M, int N,
                                int d, int64_t q_head_stride, int64_t k_head_stride,
                                int64_t q_row_stride, int64_t k_row_stride, void* stream);

/* FFI mirrors of the constexpr sizing helpers of attention_fused.h:21-45, for
 * callers that cannot evaluate C++ constexpr functions. */
size_t tilemix_routing_words_per_row_c(int N, int key_tiles_per_group);
size_t tilemix_routing_word_count_c(int M, int N, int key_tiles_per_group);
size_t tilemix_shared_bytes_c(int d, int quantized);

/* Library version string, e.g. "tilemix-hip 0.1 gfx950". */
const char* tilemix_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TILEMIX_CAPI_H */
