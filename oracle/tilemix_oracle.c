/*
 * TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT. See tilemix_oracle.h.
 *
 * Built with -ffp-contract=off on x86-64 (SSE scalar float), so every float
 * expression below is a sequence of IEEE binary32 operations rounded to
 * nearest-even, as the reference's host oracles are.
 */
#include "tilemix_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

static uint32_t float_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

static float bits_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

float tmo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    const uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0x1fu) return bits_float(sign | 0x7f800000u | (mantissa << 13));
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24, exact in binary32 */
        const float magnitude = (float)mantissa * 5.9604644775390625e-8f;
        return sign ? -magnitude : magnitude;
    }
    return bits_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

uint16_t tmo_float_to_half(float f) {
    const uint32_t x = float_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t magnitude = x & 0x7fffffffu;
    if (magnitude > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((magnitude >> 13) & 0x3ffu));
    if (magnitude >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536 or inf */
    if (magnitude < 0x38800000u) {
        /* result is a half subnormal (or zero): count units of 2^-24 */
        if (magnitude <= 0x33000000u) return sign; /* <= 2^-25 rounds to zero (tie to even) */
        const uint32_t exponent = magnitude >> 23;
        const uint32_t significand = (magnitude & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exponent; /* value = significand * 2^(exponent-150) */
        uint32_t units = significand >> shift;
        const uint32_t remainder = significand & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (remainder > halfway || (remainder == halfway && (units & 1u))) ++units;
        return (uint16_t)(sign | units);
    }
    uint32_t h = ((((magnitude >> 23) - 112u) << 10) | ((magnitude >> 13) & 0x3ffu));
    const uint32_t remainder = magnitude & 0x1fffu;
    if (remainder > 0x1000u || (remainder == 0x1000u && (h & 1u))) ++h; /* carry may reach inf */
    return (uint16_t)(sign | h);
}

void tmo_halves_to_floats(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; ++i) f[i] = tmo_half_to_float(h[i]);
}

void tmo_floats_to_halves(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = tmo_float_to_half(f[i]);
}

/* -------------------------------------------------------------- mt19937 */

void tmo_mt19937_seed(tmo_mt19937* g, uint32_t seed) {
    g->state[0] = seed;
    for (int i = 1; i < 624; ++i) {
        const uint32_t prev = g->state[i - 1];
        g->state[i] = 1812433253u * (prev ^ (prev >> 30)) + (uint32_t)i;
    }
    g->index = 624;
}

static void mt19937_twist(tmo_mt19937* g) {
    for (int i = 0; i < 624; ++i) {
        const uint32_t y = (g->state[i] & 0x80000000u) | (g->state[(i + 1) % 624] & 0x7fffffffu);
        uint32_t next = g->state[(i + 397) % 624] ^ (y >> 1);
        if (y & 1u) next ^= 0x9908b0dfu;
        g->state[i] = next;
    }
    g->index = 0;
}

uint32_t tmo_mt19937_next(tmo_mt19937* g) {
    if (g->index >= 624) mt19937_twist(g);
    uint32_t y = g->state[g->index++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

void tmo_mt19937_outputs(uint32_t seed, uint32_t* out, size_t n) {
    tmo_mt19937 g;
    tmo_mt19937_seed(&g, seed);
    for (size_t i = 0; i < n; ++i) out[i] = tmo_mt19937_next(&g);
}

/* ------------------------------------------------------- test inputs */

static void fill_half(uint16_t* x, size_t n, float value) {
    const uint16_t h = tmo_float_to_half(value);
    for (size_t i = 0; i < n; ++i) x[i] = h;
}

/* Value draw of src/tests/tilemix_test.cu:49-51: an integer in
 * [-10000, 10000] divided by 10000 in binary32, rounded to fp16. */
static uint16_t draw_value(tmo_mt19937* g) {
    const int integer = (int)(tmo_mt19937_next(g) % 20001u) - 10000;
    return tmo_float_to_half((float)integer / 10000.0f);
}

int tmo_make_inputs(int m, int n, int d, const char* pattern,
                    uint16_t* q, uint16_t* k, uint16_t* v) {
    const size_t qn = (size_t)m * (size_t)d, kn = (size_t)n * (size_t)d;
    tmo_mt19937 g;
    tmo_mt19937_seed(&g, (uint32_t)(m * 131 + n * 17 + d));
    for (size_t i = 0; i < qn; ++i) q[i] = draw_value(&g);
    for (size_t i = 0; i < kn; ++i) k[i] = draw_value(&g);
    for (size_t i = 0; i < kn; ++i) v[i] = draw_value(&g);

    if (strcmp(pattern, "random") == 0) return 0;
    if (strcmp(pattern, "zeros") == 0) {
        fill_half(q, qn, 0.0f);
        fill_half(k, kn, 0.0f);
        fill_half(v, kn, 0.0f);
        return 0;
    }
    if (strcmp(pattern, "block-outliers") == 0) {
        if (m < 129 || n < 129) return -1;
        q[(size_t)127 * d] = tmo_float_to_half(8.0f);
        q[(size_t)128 * d] = tmo_float_to_half(0.125f);
        k[(size_t)63 * d] = tmo_float_to_half(-16.0f);
        k[(size_t)128 * d] = tmo_float_to_half(0.25f);
        return 0;
    }
    if (strcmp(pattern, "max-int8") == 0) {
        fill_half(q, qn, 1.0f);
        fill_half(k, kn, 1.0f);
        fill_half(k, (size_t)d, -1.0f);
        return 0;
    }
    if (strcmp(pattern, "zero-v") == 0) {
        fill_half(v, kn, 0.0f);
        return 0;
    }
    if (strcmp(pattern, "constant-v") == 0) {
        for (int key = 0; key < n; ++key)
            for (int f = 0; f < d; ++f)
                v[(size_t)key * d + f] = tmo_float_to_half((float)(f % 7 - 3) * 0.25f);
        return 0;
    }
    if (strcmp(pattern, "cancellation") == 0) {
        fill_half(q, qn, 0.0f);
        for (int key = 0; key < n; ++key)
            for (int f = 0; f < d; ++f)
                v[(size_t)key * d + f] = tmo_float_to_half(key % 2 ? -1.0f : 1.0f);
        return 0;
    }
    if (strcmp(pattern, "large-dot") == 0) {
        fill_half(q, qn, 1000.0f);
        fill_half(k, kn, -1000.0f);
        fill_half(k, (size_t)d, 1000.0f);
        return 0;
    }
    fill_half(q, qn, 0.0f);
    if (strcmp(pattern, "uniform") == 0) return 0;

    /* Closed-form score patterns: only feature 0 of Q and K is non-zero. */
    const int rising = strcmp(pattern, "rising") == 0;
    const int falling = strcmp(pattern, "falling") == 0;
    const int alternating = strcmp(pattern, "alternating") == 0;
    const int late = strcmp(pattern, "late-extreme") == 0;
    const int negative = strcmp(pattern, "negative") == 0;
    if (!(rising || falling || alternating || late || negative)) return -1;
    if (alternating && (n - 1) / 32 >= 5) return -1;
    fill_half(k, kn, 0.0f);
    for (int query = 0; query < m; ++query) q[(size_t)query * d] = tmo_float_to_half(1.0f);
    static const float alt_scores[5] = {0.0f, 4.0f, -2.0f, 8.0f, 10.0f};
    static const float alt_values[5] = {1.0f, -1.0f, 2.0f, -2.0f, 3.0f};
    for (int key = 0; key < n; ++key) {
        const int tile = key / 32;
        float score, value;
        if (rising || falling) {
            score = rising ? 4.0f * (float)(tile - 1) : 4.0f * (float)(1 - tile);
            value = tile == 0 ? 1.0f : (tile == 1 ? -1.0f : 2.0f);
        } else if (alternating) {
            score = alt_scores[tile];
            value = alt_values[tile];
        } else if (late) {
            score = key == n - 1 ? 1000.0f : 0.0f;
            value = key == n - 1 ? 3.0f : 1.0f;
        } else {
            score = -1000.0f;
            value = (float)(key % 7 - 3) * 0.25f;
        }
        k[(size_t)key * d] = tmo_float_to_half(score);
        for (int f = 0; f < d; ++f) v[(size_t)key * d + f] = tmo_float_to_half(value);
    }
    return 0;
}

/* ------------------------------------------------------------ quantizer */

void tmo_quantize(const uint16_t* x, int rows, int d, int block_rows,
                  int8_t* out, uint16_t* scales) {
    for (int first = 0; first < rows; first += block_rows) {
        const int last = rows < first + block_rows ? rows : first + block_rows;
        float maximum = 0.0f;
        for (int row = first; row < last; ++row)
            for (int f = 0; f < d; ++f) {
                const float a = fabsf(tmo_half_to_float(x[(size_t)row * d + f]));
                if (a > maximum) maximum = a;
            }
        const float scale = maximum / 127.0f; /* binary32 division, round to nearest */
        scales[first / block_rows] = tmo_float_to_half(scale);
        for (int row = first; row < last; ++row)
            for (int f = 0; f < d; ++f) {
                const size_t index = (size_t)row * d + f;
                const float normalized = scale == 0.0f ? 0.0f : tmo_half_to_float(x[index]) / scale;
                const float shifted = normalized < 0.0f ? normalized - 0.5f : normalized + 0.5f;
                /* __float2int_rz (src/tilemix.cu:45): truncation toward zero, NaN
                   (x NaN, or x = +-inf in a block whose maximum is inf) -> 0;
                   C's (int) of a NaN is undefined, so that case is spelled out. */
                int rounded = shifted != shifted ? 0 : (int)shifted;
                if (rounded > 127) rounded = 127;
                if (rounded < -127) rounded = -127;
                out[index] = (int8_t)rounded;
            }
    }
}

int32_t tmo_int8_dot(const int8_t* q8, const int8_t* k8, int query, int key, int d) {
    int64_t sum = 0;
    for (int f = 0; f < d; ++f)
        sum += (int64_t)q8[(size_t)query * d + f] * (int64_t)k8[(size_t)key * d + f];
    return (int32_t)sum;
}

/* ------------------------------------------------------ tilemix (fp64) */

static void tilemix_row(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const int8_t* q8, const int8_t* k8,
                        const uint16_t* q_scales, const uint16_t* k_scales,
                        const uint8_t* routes, int N, int d, float score_scale, int causal,
                        int query, double* scores, double* out_row) {
    const int key_tiles = (N + 31) / 32;
    double maximum = -INFINITY;
    for (int key = 0; key < N; ++key) {
        const int route = routes ? routes[(size_t)(query / 16) * key_tiles + key / 32] : 0;
        if (route == 2 || (causal && key > query)) {
            scores[key] = -INFINITY;
            continue;
        }
        double dot = 0.0;
        if (route == 1) {
            dot = (double)tmo_int8_dot(q8, k8, query, key, d);
            dot *= (double)tmo_half_to_float(q_scales[query / 128]);
            dot *= (double)tmo_half_to_float(k_scales[key / 64]);
        } else {
            for (int f = 0; f < d; ++f)
                dot += (double)tmo_half_to_float(q[(size_t)query * d + f])
                     * (double)tmo_half_to_float(k[(size_t)key * d + f]);
        }
        scores[key] = dot * (double)score_scale;
        if (scores[key] > maximum) maximum = scores[key];
    }
    for (int f = 0; f < d; ++f) out_row[f] = 0.0;
    if (maximum == -INFINITY) return; /* no visible key */
    double denominator = 0.0;
    for (int key = 0; key < N; ++key) {
        scores[key] = exp(scores[key] - maximum);
        denominator += scores[key];
    }
    for (int key = 0; key < N; ++key) {
        const double probability = scores[key] / denominator;
        if (probability == 0.0) continue;
        for (int f = 0; f < d; ++f)
            out_row[f] += probability * (double)tmo_half_to_float(v[(size_t)key * d + f]);
    }
}

void tmo_tilemix(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const int8_t* q8, const int8_t* k8,
                 const uint16_t* q_scales, const uint16_t* k_scales,
                 const uint8_t* routes, int M, int N, int d, float score_scale,
                 int causal, const int32_t* rows, int nrows, double* out) {
    const int count = rows ? nrows : M;
#pragma omp parallel
    {
        double* scores = (double*)malloc(sizeof(double) * (size_t)N);
#pragma omp for schedule(dynamic, 4)
        for (int i = 0; i < count; ++i) {
            const int query = rows ? rows[i] : i;
            tilemix_row(q, k, v, q8, k8, q_scales, k_scales, routes, N, d, score_scale,
                        causal, query, scores, out + (size_t)i * d);
        }
        free(scores);
    }
}

/* ------------------------------------------------ dense attention (fp64) */

int tmo_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  int M, int N, int d, double* out) {
    const double scale = 1.0 / sqrt((double)d);
    for (size_t i = 0; i < (size_t)M * d; ++i)
        if (!isfinite(tmo_half_to_float(q[i]))) return -1;
    for (size_t i = 0; i < (size_t)N * d; ++i)
        if (!isfinite(tmo_half_to_float(k[i])) || !isfinite(tmo_half_to_float(v[i]))) return -1;
    double* weights = (double*)malloc(sizeof(double) * (size_t)N);
    for (int query = 0; query < M; ++query) {
        double maximum = -INFINITY;
        for (int key = 0; key < N; ++key) {
            double dot = 0.0;
            for (int f = 0; f < d; ++f)
                dot += (double)tmo_half_to_float(q[(size_t)query * d + f])
                     * (double)tmo_half_to_float(k[(size_t)key * d + f]);
            weights[key] = dot * scale;
            if (weights[key] > maximum) maximum = weights[key];
        }
        double denominator = 0.0;
        for (int key = 0; key < N; ++key) {
            weights[key] = exp(weights[key] - maximum);
            denominator += weights[key];
        }
        double* row = out + (size_t)query * d;
        for (int f = 0; f < d; ++f) row[f] = 0.0;
        for (int key = 0; key < N; ++key) {
            const double probability = weights[key] / denominator;
            for (int f = 0; f < d; ++f)
                row[f] += probability * (double)tmo_half_to_float(v[(size_t)key * d + f]);
        }
    }
    free(weights);
    return 0;
}

/* ------------------------------------------------------- route decoding */

void tmo_decode_routes(const uint64_t* route_words, const uint64_t* skip_words,
                       int M, int N, int key_tiles_per_group, uint8_t* routes) {
    const size_t query_tiles = ((size_t)M + 15) / 16;
    const size_t key_tiles = ((size_t)N + 31) / 32;
    const size_t groups = (key_tiles + (size_t)key_tiles_per_group - 1) / (size_t)key_tiles_per_group;
    const size_t words_per_row = (groups + 63) / 64;
    for (size_t row = 0; row < query_tiles; ++row)
        for (size_t tile = 0; tile < key_tiles; ++tile) {
            const size_t group = tile / (size_t)key_tiles_per_group;
            const size_t word = row * words_per_row + group / 64;
            const unsigned bit = (unsigned)(group % 64);
            uint8_t code = 0;
            if (route_words && ((route_words[word] >> bit) & 1u)) code = 1;
            if (skip_words && ((skip_words[word] >> bit) & 1u)) code = 2;
            routes[row * key_tiles + tile] = code;
        }
}
