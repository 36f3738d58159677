// Exhaustive device check of the quantizer's division-free quotient
// (tilemix_device.h: quotient / quantize_value_recip / quantize_in_block /
// quantize_half) against IEEE division (quantize_value, built with
// -fhip-fp32-correctly-rounded-divide-sqrt): for every positive finite fp16
// block maximum a and every fp16 x with |x| <= a, the fp32 quotients (as
// values) and the int8 results must agree; quantize_half reads x from either
// half of a word whose other half holds a different value. Also checks
// pack_bytes against shifts for every int8 value in each byte position.
// Prints "PASS <pairs>" or the first mismatches; exit code 0 on pass.
#include "tilemix_device.h"

#include <cstdio>

using namespace tilemix;

__global__ void check(unsigned long long* pairs, unsigned long long* bad, unsigned* first) {
    const unsigned a_bits = blockIdx.x + 1;  // 0x0001 .. 0x7bff: positive finite fp16
    if (a_bits > 0x7bffu) return;
    const float absmax = half_bits_to_float(static_cast<std::uint16_t>(a_bits));
    const float scale = block_scale(absmax);
    const float recip = 1.0f / scale;
    unsigned long long n = 0, wrong = 0;
    // x over all fp16 bit patterns with |x| <= absmax (magnitude bits <= a_bits), both signs.
    for (unsigned m = threadIdx.x; m <= a_bits; m += blockDim.x) {
        for (unsigned sign = 0; sign < 2; ++sign) {
            const float x = half_bits_to_float(static_cast<std::uint16_t>(m | (sign << 15)));
            const float exact = x / scale;
            const float fast = quotient(x, scale, recip);
            const int q_exact = quantize_value(x, scale);
            const int q_fast = quantize_value_recip(x, scale, recip);
            const int q_block = quantize_in_block(x, scale, recip);
            const unsigned bits = m | (sign << 15), other = bits ^ 0x5a5au;
            const int q_lo = quantize_half<0>(bits | (other << 16), scale, recip);
            const int q_hi = quantize_half<1>(other | (bits << 16), scale, recip);
            ++n;
            // Quotients compare as floats: x = -0 gives -0 by division and +0 here,
            // which quantize alike; every other quotient must match bit for bit.
            if (exact != fast || q_exact != q_fast || q_exact != q_block || q_exact != q_lo || q_exact != q_hi) {
                ++wrong;
                if (atomicCAS(first, 0u, (a_bits << 16) | m | (sign << 15)) == 0u) {}
            }
        }
    }
    if (blockIdx.x == 0) {
        // pack_bytes: every int8 value in each position beside distinct neighbours.
        for (int v = -128 + static_cast<int>(threadIdx.x); v < 128; v += blockDim.x) {
            const int a = v, b = -v - 1, c = v ^ 0x55, d = 127 - v;
            const std::uint32_t shifted = (static_cast<std::uint32_t>(a) & 0xffu) |
                                          ((static_cast<std::uint32_t>(b) & 0xffu) << 8) |
                                          ((static_cast<std::uint32_t>(c) & 0xffu) << 16) |
                                          (static_cast<std::uint32_t>(d) << 24);
            ++n;
            if (pack_bytes(a, b, c, d) != shifted || pack_bytes(d, c, b, a) != __builtin_bswap32(shifted)) {
                ++wrong;
                (void)atomicCAS(first, 0u, 0xffff0000u | (static_cast<unsigned>(v) & 0xffffu));
            }
        }
    }
    atomicAdd(pairs, n);
    if (wrong) atomicAdd(bad, wrong);
}

int main() {
    unsigned long long *pairs, *bad;
    unsigned* first;
    if (hipMalloc(&pairs, 8) != hipSuccess || hipMalloc(&bad, 8) != hipSuccess || hipMalloc(&first, 4) != hipSuccess) {
        std::puts("FAIL allocation");
        return 2;
    }
    (void)hipMemset(pairs, 0, 8);
    (void)hipMemset(bad, 0, 8);
    (void)hipMemset(first, 0, 4);
    check<<<0x7bff, 256>>>(pairs, bad, first);
    unsigned long long n = 0, wrong = 0;
    unsigned f = 0;
    if (hipMemcpy(&n, pairs, 8, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(&wrong, bad, 8, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(&f, first, 4, hipMemcpyDeviceToHost) != hipSuccess) {
        std::puts("FAIL copy");
        return 2;
    }
    (void)hipFree(pairs);
    (void)hipFree(bad);
    (void)hipFree(first);
    if (wrong) {
        std::printf("FAIL %llu of %llu pairs differ (first: absmax bits 0x%04x, x bits 0x%04x)\n", wrong, n, f >> 16, f & 0xffffu);
        return 1;
    }
    std::printf("PASS %llu pairs\n", n);
    return 0;
}
