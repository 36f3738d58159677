#ifndef TILEMIX_ORACLE_H
#define TILEMIX_ORACLE_H
/*
 * TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.
 *
 * CPU restatement (plain C99) of the reference's TileMix semantics, used only
 * by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. The shipped library never links or calls it.
 *
 * What each function follows (paths relative to the reference repository):
 *   tmo_quantize      src/tests/reference_tilemix.h:16-41 (and the kernel
 *                     src/tilemix.cu:16-49 it mirrors)
 *   tmo_int8_dot      src/tests/reference_tilemix.h:43-51
 *   tmo_tilemix       src/tests/reference_tilemix.h:53-90, extended with a
 *                     skip route and a causal mask (no reference counterpart)
 *   tmo_attention     src/tests/reference_attention.h:12-52
 *   tmo_make_inputs   src/tests/tilemix_test.cu:43-134
 *   tmo_decode_routes src/tilemix.cu:99-106 (mask decode / decoded_bits)
 *   tmo_mt19937_*     std::mt19937 as used by src/tests/tilemix_test.cu:48
 *   tmo_half_*        IEEE binary16 <-> binary32, round-to-nearest-even
 *                     (__float2half / __half2float semantics)
 *
 * How each is pinned is recorded in the tests that import it.
 */
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float tmo_half_to_float(uint16_t h);
uint16_t tmo_float_to_half(float f);
void tmo_halves_to_floats(const uint16_t* h, float* f, size_t n);
void tmo_floats_to_halves(const float* f, uint16_t* h, size_t n);

typedef struct tmo_mt19937 {
    uint32_t state[624];
    int index;
} tmo_mt19937;
void tmo_mt19937_seed(tmo_mt19937* g, uint32_t seed);
uint32_t tmo_mt19937_next(tmo_mt19937* g);
/* Fills out[0..n) with consecutive outputs of std::mt19937(seed). */
void tmo_mt19937_outputs(uint32_t seed, uint32_t* out, size_t n);

/* Returns 0, or -1 for an unknown pattern / unmet precondition. */
int tmo_make_inputs(int m, int n, int d, const char* pattern,
                    uint16_t* q, uint16_t* k, uint16_t* v);

void tmo_quantize(const uint16_t* x, int rows, int d, int block_rows,
                  int8_t* out, uint16_t* scales);

int32_t tmo_int8_dot(const int8_t* q8, const int8_t* k8, int query, int key, int d);

/* routes[qtile * ceil(N/32) + ktile] in {0 = FP16, 1 = INT8, 2 = skip};
 * routes == NULL means every cell is FP16. rows == NULL computes every row
 * into out[M*d]; otherwise row rows[i] goes to out[i*d]. A row without any
 * visible key yields zeros. */
void tmo_tilemix(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const int8_t* q8, const int8_t* k8,
                 const uint16_t* q_scales, const uint16_t* k_scales,
                 const uint8_t* routes, int M, int N, int d, float score_scale,
                 int causal, const int32_t* rows, int nrows, double* out);

/* Dense softmax(Q K^T / sqrt(d)) V in double. Returns -1 on non-finite input. */
int tmo_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  int M, int N, int d, double* out);

/* Decodes packed route words (and optional skip words, same packing) into one
 * code per 16x32 cell, as the kernel's routing trace defines it. */
void tmo_decode_routes(const uint64_t* route_words, const uint64_t* skip_words,
                       int M, int N, int key_tiles_per_group, uint8_t* routes);

#ifdef __cplusplus
}
#endif
#endif
