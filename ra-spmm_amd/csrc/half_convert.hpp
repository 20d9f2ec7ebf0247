// half_convert.hpp — IEEE-754 binary32 -> binary16 / bfloat16 conversions,
// round to nearest, ties to even, written from the standard's definition.
// Shared by the host and the device tile-format builders so both store
// bit-identical values.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ra {

__host__ __device__ inline uint32_t float_bits(float f) {
    union {
        float f;
        uint32_t u;
    } c;
    c.f = f;
    return c.u;
}

__host__ __device__ inline uint16_t half_rne_bits(float f) {
    const uint32_t x = float_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u)  // inf / nan (nan stays quiet)
        return static_cast<uint16_t>(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u | ((a >> 13) & 0x3FFu) : 0u));
    if (a >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // >= 65520 -> inf
    if (a < 0x38800000u) {                                                // below 2^-14: subnormal
        if (a < 0x33000000u) return static_cast<uint16_t>(sign);          // <= 2^-25 -> 0
        const uint32_t e = a >> 23;
        const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;  // value in units of 2^-24
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return static_cast<uint16_t>(sign | q);
    }
    uint32_t q = (a >> 13) - (112u << 10);  // rebias exponent 127 -> 15
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;  // carry may reach inf: correct
    return static_cast<uint16_t>(sign | q);
}

__host__ __device__ inline uint16_t bf16_rne_bits(float f) {
    const uint32_t x = float_bits(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    return static_cast<uint16_t>((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

}  // namespace ra
