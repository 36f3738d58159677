#pragma once
// Device-side building blocks shared by the gfx950 TileMix kernels.
//
// Build requirements (set by tilemix-cuda_amd/build.py): --offload-arch=gfx950,
// -fhip-fp32-correctly-rounded-divide-sqrt (binary32 '/' is IEEE
// round-to-nearest, which the quantizer's bit-exact contract depends on) and no
// fast-math flags.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace tilemix {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef unsigned int uint4v __attribute__((ext_vector_type(4)));
typedef unsigned int uint2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

inline constexpr int kWave = 64;

__device__ __forceinline__ float half_bits_to_float(std::uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// binary32 -> binary16, round to nearest even (v_cvt_f16_f32 in the default
// rounding mode), matching __float2half_rn.
__device__ __forceinline__ std::uint16_t float_to_half_bits(float value) {
    return __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(value));
}

// Symmetric INT8 quantization of one element (reference src/tilemix.cu:44-46):
// the IEEE quotient by the fp32 block scale, a binary32 add of +-0.5, then
// truncation toward zero and a clamp to [-127, 127]. Keeping the rounded add
// (rather than an exact round-half-away) is part of the bit-exact contract.
__device__ __forceinline__ int quantize_value(float x, float scale) {
    const float normalized = scale > 0.0f ? x / scale : 0.0f;
    const float shifted = normalized + __builtin_copysignf(0.5f, normalized);
    const int rounded = static_cast<int>(shifted);
    return rounded < -127 ? -127 : (rounded > 127 ? 127 : rounded);
}

// Block scale: fp32 absmax / 127 with IEEE rounding (src/tilemix.cu:37).
__device__ __forceinline__ float block_scale(float absmax) { return absmax / 127.0f; }

// x / scale rounded to nearest without a division per element (Markstein's
// correction step): with recip = RN(1 / scale), y = RN(x * recip) is within
// an ulp of the quotient, the fma gives its exact remainder, and one more fma
// rounds to the correctly rounded quotient. The operands here are always
// well scaled (|x| <= absmax = 127 * scale, scale a normal float or 0), and
// the result equals IEEE x / scale for every fp16 x and fp16 absmax; the
// exhaustive device check in tests/native/quant_division_check.hip pins that.
__device__ __forceinline__ float quotient(float x, float scale, float recip) {
    const float y = x * recip;
    const float r = __builtin_fmaf(-scale, y, x);
    return __builtin_fmaf(r, recip, y);
}

// quantize_value with the per-block reciprocal (recip = 1 / scale, any value
// when scale == 0): the same bytes as quantize_value.
__device__ __forceinline__ int quantize_value_recip(float x, float scale, float recip) {
    const float normalized = scale > 0.0f ? quotient(x, scale, recip) : 0.0f;
    const float shifted = normalized + __builtin_copysignf(0.5f, normalized);
    const int rounded = static_cast<int>(shifted);
    return rounded < -127 ? -127 : (rounded > 127 ? 127 : rounded);
}

// quantize_value_recip for an element of its own block with a positive scale
// (|x| <= absmax, scale = absmax / 127 > 0): |x / scale| <= 127 (1 + 2^-24),
// so the shifted quotient truncates into [-127, 127] and the clamp is never
// taken; a NaN quotient converts to 0 either way. The exhaustive device check
// in tests/native/quant_division_check.hip compares it with quantize_value.
__device__ __forceinline__ int quantize_in_block(float x, float scale, float recip) {
    const float normalized = quotient(x, scale, recip);
    return static_cast<int>(normalized + __builtin_copysignf(0.5f, normalized));
}

// quantize_in_block of half kHalf (0 = low) of two packed fp16 elements. The
// first product is read straight from the fp16 half (v_fma_mix_f32 with a
// zero addend: RN(x * recip), which differs from the f32 product only in the
// sign of a zero product, and a zero quotient rounds to 0 either way); the
// exhaustive device check in tests/native/quant_division_check.hip compares
// both halves with quantize_value.
template <int kHalf>
__device__ __forceinline__ int quantize_half(std::uint32_t pair, float scale, float recip) {
    float y;
    if constexpr (kHalf == 0)
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(pair), "v"(recip));
    else
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(y) : "v"(pair), "v"(recip));
    const float x = half_bits_to_float(static_cast<std::uint16_t>(pair >> (16 * kHalf)));
    const float q = __builtin_fmaf(__builtin_fmaf(-scale, y, x), recip, y);
    return static_cast<int>(q + __builtin_copysignf(0.5f, q));
}

// Elementwise unsigned maximum of two pairs of 16-bit values.
__device__ __forceinline__ unsigned max_u16x2(unsigned a, unsigned b) {
    unsigned r;
    asm("v_pk_max_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Maximum over the wave's 64 lanes, returned in every lane: DPP steps inside
// rows of 16 lanes (quad partners ^1 and ^2, then the mirrored lane within 8
// and within 16), then v_permlane16_swap / v_permlane32_swap across rows
// (inline assembly, s_nop 1 covering the VALU-write -> permlane-read hazard).
__device__ __forceinline__ unsigned wave_max_bits(unsigned v) {
    v = max(v, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, false)));
    v = max(v, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, false)));
    v = max(v, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xf, 0xf, false)));
    v = max(v, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xf, 0xf, false)));
    unsigned a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    v = max(a, b);
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return max(a, b);
}

__device__ __forceinline__ float wave_max(float value) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) value = fmaxf(value, __shfl_xor(value, offset));
    return value;
}

// Packs four quantized values (low byte first) into one 32-bit word.
// Three v_perm_b32: (a, b) and (c, d) low bytes into halves, then the halves.
__device__ __forceinline__ std::uint32_t pack_bytes(int a, int b, int c, int d) {
    const std::uint32_t lo = __builtin_amdgcn_perm(static_cast<std::uint32_t>(b), static_cast<std::uint32_t>(a), 0x0c0c0400u);
    const std::uint32_t hi = __builtin_amdgcn_perm(static_cast<std::uint32_t>(d), static_cast<std::uint32_t>(c), 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

}  // namespace tilemix
