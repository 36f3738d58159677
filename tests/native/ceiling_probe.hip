// Hardware ceilings that bound the attention kernel on MI355X (gfx950).
//
// Three measurements, each printed as one JSON line:
//
//  * mfma_rate: sustained 32x32 MFMA throughput (v_mfma_f32_32x32x16_f16 or
//    v_mfma_i32_32x32x32_i8, four independent accumulator chains per wave,
//    two waves per SIMD on every CU) for operand data that is all zero or
//    random. The card runs at its power limit under MFMA load, and how far
//    its clock falls below the 2.4 GHz that the published peaks assume
//    depends on how many operand bits toggle.
//  * lds_rate: LDS read throughput per CU for the two fragment reads the
//    attention kernel uses (ds_read_b128 for K / K8, ds_read_b64_tr_b16 for
//    V^T).
//  * phase_rate: the attention kernel's two MFMA phases with zero operands
//    (so the clock stays near 2.4 GHz): the score phase (16 MFMAs on two
//    accumulator chains, K fragments read two chunks ahead) and the P.V
//    phase (16 MFMAs on four chains, V^T fragments read three steps ahead),
//    alone and together with the kernel's two workgroup barriers per tile.
//
// Fractions are of the 2.4 GHz rate (one 32x32 MFMA per 32 clocks per SIMD).
// Usage: ceiling_probe [--quick]
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int16v __attribute__((ext_vector_type(16)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

constexpr int kGroups = 512;      // two 4-wave workgroups per CU on 256 CUs
constexpr int kThreads = 256;
constexpr double kPeakClock = 2.4e9;

#define CHECK(call)                                                                          \
    do {                                                                                     \
        const hipError_t status_ = (call);                                                   \
        if (status_ != hipSuccess) {                                                         \
            std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(status_));      \
            std::exit(1);                                                                    \
        }                                                                                    \
    } while (0)

// Four independent accumulator chains; operands are read from `words`
// (8 dwords per thread) so that the data decides how many bits toggle.
template <bool kInt8>
__global__ __launch_bounds__(kThreads, 2) void mfma_rate(const std::uint32_t* words, float* sink, int iterations) {
    const std::uint32_t* w = words + ((blockIdx.x * kThreads + threadIdx.x) & 4095) * 8;
    const int4v a0{static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]), static_cast<int>(w[3])};
    const int4v a1{static_cast<int>(w[4]), static_cast<int>(w[5]), static_cast<int>(w[6]), static_cast<int>(w[7])};
    const int4v b0{a1[3], a1[2], a1[1], a1[0]};
    const int4v b1{a0[3], a0[2], a0[1], a0[0]};
    float16v f[4] = {};
    int16v n[4] = {};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int4v a = (c & 1) ? a1 : a0, b = (c & 2) ? b1 : b0;
            if constexpr (kInt8)
                n[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, n[c], 0, 0, 0);
            else
                f[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b),
                                                              f[c], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s += kInt8 ? static_cast<float>(n[c][0] + n[c][9]) : f[c][0] + f[c][9];
    sink[blockIdx.x * kThreads + threadIdx.x] = s;
}

// Every wave reads 8 KiB of a zeroed 32 KiB LDS buffer per iteration,
// conflict-free, as 8 ds_read_b128 or 16 ds_read_b64_tr_b16.
template <bool kTransposed>
__global__ __launch_bounds__(kThreads, 2) void lds_rate(float* sink, int iterations) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[32768];
    for (int e = threadIdx.x; e < 32768 / 4; e += kThreads) reinterpret_cast<int*>(lds)[e] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int acc = 0;
    for (int it = 0; it < iterations; ++it) {
        asm volatile("" ::: "memory");  // the buffer may have changed: read it again
        if constexpr (kTransposed) {
            short4v r[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int offset = ((u * 4 + wave) * 512 + (lane & 15) * 8 + (lane >> 4) * 128) & 32767;
                r[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lds + offset));
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) acc += r[u][0] + r[u][3];
        } else {
            int4v r[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int offset = ((u * 4 + wave) * 1024 + lane * 16) & 32767;
                r[u] = *reinterpret_cast<const int4v*>(lds + offset);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += r[u][0] + r[u][3];
        }
    }
    sink[blockIdx.x * kThreads + threadIdx.x] = static_cast<float>(acc);
}

// The attention kernel's MFMA phases over zeroed 64-key K and V tiles with
// 256-byte rows laid out as the kernel lays them (16-byte chunks rotated by
// row). kPhase: 0 scores, 1 P.V, 2 scores + barrier + P.V + barrier.
template <int kPhase>
__global__ __launch_bounds__(kThreads, 2) void phase_rate(float* sink, int iterations) {
    __shared__ __attribute__((aligned(16))) unsigned char lds_k[16384];
    __shared__ __attribute__((aligned(16))) unsigned char lds_v[16384];
    for (int e = threadIdx.x; e < 4096; e += kThreads) {
        reinterpret_cast<int*>(lds_k)[e] = 0;
        reinterpret_cast<int*>(lds_v)[e] = 0;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, q = lane & 31, h = lane >> 5, i = lane & 15;
    int k_lane[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) k_lane[c] = q * 256 + ((((2 * c + h) + q) & 15) << 4);
    int v_lane[4];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb) {
        const int row = 4 * h + (i >> 2);
        const int byte = 2 * (16 * fb + 64 * ((lane >> 4) & 1) + 4 * (i & 3));
        v_lane[fb] = row * 256 + ((((byte >> 4) + 2 * row) & 15) << 4) + (byte & 15);
    }
    half8 qf[8] = {};
    half8 p[4] = {};
    float16v s[2] = {};
    float16v o[4] = {};
    for (int it = 0; it < iterations; ++it) {
        asm volatile("" ::: "memory");
        if constexpr (kPhase != 1) {
            half8 kf[3][2];
            auto load = [&](int c, half8 (&dst)[2]) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    dst[kb] = *reinterpret_cast<const half8*>(lds_k + 32 * 256 * kb + k_lane[c]);
            };
            load(0, kf[0]);
            load(1, kf[1]);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if (c + 2 < 8) load(c + 2, kf[(c + 2) % 3]);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c % 3][kb], qf[c], s[kb], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (kPhase == 2) __syncthreads();
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) p[ks][e] = static_cast<_Float16>(s[ks >> 1][8 * (ks & 1) + e]);
        }
        if constexpr (kPhase != 0) {
            auto v_frag = [&](int t) {
                const unsigned char* lo = lds_v + 16 * 256 * (t / 4) + v_lane[t % 4];
                const short4v a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lo));
                const short4v b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lo + 8 * 256));
                return __builtin_bit_cast(half8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            half8 vf[4];
#pragma unroll
            for (int t = 0; t < 3; ++t) vf[t] = v_frag(t);
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                if (t + 3 < 16) vf[(t + 3) % 4] = v_frag(t + 3);
                o[t % 4] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[t % 4], p[t / 4], o[t % 4], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (kPhase == 2) __syncthreads();
        }
    }
    float r = s[0][1] + s[1][2];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb) r += o[fb][0];
    sink[blockIdx.x * kThreads + threadIdx.x] = r;
}

std::uint32_t lcg(std::uint32_t& state) {
    state = state * 1664525u + 1013904223u;
    return state;
}

// Best of `reps` timed launches after `warm` untimed ones, in ms.
template <typename Launch>
float time_best(Launch launch, int warm, int reps) {
    hipEvent_t start, stop;
    CHECK(hipEventCreate(&start));
    CHECK(hipEventCreate(&stop));
    for (int w = 0; w < warm; ++w) launch();
    float best = 1e30f;
    for (int r = 0; r < reps; ++r) {
        CHECK(hipEventRecord(start));
        launch();
        CHECK(hipEventRecord(stop));
        CHECK(hipEventSynchronize(stop));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, start, stop));
        best = ms < best ? ms : best;
    }
    CHECK(hipEventDestroy(start));
    CHECK(hipEventDestroy(stop));
    return best;
}

}  // namespace

int main(int argc, char** argv) {
    const bool quick = argc > 1 && std::strcmp(argv[1], "--quick") == 0;
    const int warm = quick ? 40 : 150, reps = quick ? 5 : 10;
    std::uint32_t* words = nullptr;
    float* sink = nullptr;
    CHECK(hipMalloc(&words, 4096 * 8 * sizeof(std::uint32_t)));
    CHECK(hipMalloc(&sink, kGroups * kThreads * sizeof(float)));
    std::vector<std::uint32_t> host(4096 * 8);

    // mfma_rate: 20000 iterations x 4 MFMAs per wave, two waves per SIMD.
    const int mfma_iterations = 20000;
    struct Data { const char* name; int kind; bool int8; } cases[] = {
        {"zeros", 0, false}, {"zeros", 0, true}, {"fp16 |x| in [0.5, 4), random sign and mantissa", 1, false},
        {"fp16 |x| in [2^-11, 2^-8), random sign and mantissa", 2, false}, {"int8 random bytes", 3, true}};
    for (const Data& c : cases) {
        std::uint32_t state = 12345;
        for (std::uint32_t& word : host) {
            word = 0;
            if (c.kind == 3) {
                word = lcg(state);
            } else if (c.kind != 0) {
                for (int half = 0; half < 2; ++half) {
                    const std::uint32_t r = lcg(state);
                    const std::uint32_t exponent = (c.kind == 1 ? 14u : 4u) + (r >> 20) % 3u;
                    word |= (((r >> 31) << 15) | (exponent << 10) | (r & 0x3ffu)) << (16 * half);
                }
            }
        }
        CHECK(hipMemcpy(words, host.data(), host.size() * sizeof(std::uint32_t), hipMemcpyHostToDevice));
        const float ms = time_best([&] {
            if (c.int8) mfma_rate<true><<<kGroups, kThreads>>>(words, sink, mfma_iterations);
            else mfma_rate<false><<<kGroups, kThreads>>>(words, sink, mfma_iterations);
        }, warm, reps);
        const double per_simd = 2.0 * 4.0 * mfma_iterations;
        std::printf("{\"probe\": \"mfma_rate\", \"mfma\": \"%s\", \"operands\": \"%s\", \"ms\": %.4f, "
                    "\"frac_of_2400MHz_peak\": %.4f}\n",
                    c.int8 ? "v_mfma_i32_32x32x32_i8" : "v_mfma_f32_32x32x16_f16", c.name, ms,
                    per_simd * 32.0 / (ms * 1e-3 * kPeakClock));
    }

    const int lds_iterations = 4000;
    for (int transposed = 0; transposed < 2; ++transposed) {
        const float ms = time_best([&] {
            if (transposed) lds_rate<true><<<kGroups, kThreads>>>(sink, lds_iterations);
            else lds_rate<false><<<kGroups, kThreads>>>(sink, lds_iterations);
        }, warm, reps);
        const double bytes_per_cu = 8.0 * 8192.0 * lds_iterations;  // 8 waves x 8 KiB per iteration
        std::printf("{\"probe\": \"lds_rate\", \"read\": \"%s\", \"ms\": %.4f, \"bytes_per_clk_per_cu_at_2400MHz\": %.1f}\n",
                    transposed ? "ds_read_b64_tr_b16" : "ds_read_b128", ms, bytes_per_cu / (ms * 1e-3) / kPeakClock);
    }

    const int phase_iterations = 2000;
    const char* phases[] = {"scores: 16 MFMAs, 2 chains, K ds_read_b128 two chunks ahead",
                            "P.V: 16 MFMAs, 4 chains, V^T ds_read_b64_tr_b16 three steps ahead",
                            "scores + barrier + P.V + barrier (one tile)"};
    for (int phase = 0; phase < 3; ++phase) {
        const float ms = time_best([&] {
            if (phase == 0) phase_rate<0><<<kGroups, kThreads>>>(sink, phase_iterations);
            else if (phase == 1) phase_rate<1><<<kGroups, kThreads>>>(sink, phase_iterations);
            else phase_rate<2><<<kGroups, kThreads>>>(sink, phase_iterations);
        }, warm, reps);
        const double per_simd = 2.0 * (phase == 2 ? 32.0 : 16.0) * phase_iterations;
        std::printf("{\"probe\": \"phase_rate\", \"phase\": \"%s\", \"operands\": \"zeros\", \"ms\": %.4f, "
                    "\"frac_of_2400MHz_peak\": %.4f}\n",
                    phases[phase], ms, per_simd * 32.0 / (ms * 1e-3 * kPeakClock));
    }
    CHECK(hipDeviceSynchronize());
    CHECK(hipFree(words));
    CHECK(hipFree(sink));
    return 0;
}
