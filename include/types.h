/* types.h — scalar types shared by the reference-signature headers.
 *
 * Mirrors the echo-core interface include/types.h:1-43 (fp16_t as raw IEEE
 * half bits, 64-byte alignment macro, half <-> float helpers) so that code
 * written against it compiles unchanged.  The conversions here are portable
 * C++: decode is exact, encode rounds to nearest even, as the reference's F16C
 * intrinsics do (_cvtsh_ss / _cvtss_sh(f, 0)). */
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>

using fp16_t = uint16_t;

constexpr size_t CACHE_LINE_SIZE = 64;

#define EC_ALIGN alignas(64)

inline float fp16_to_fp32(fp16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);  // inf / nan
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  // subnormal half: normalise
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while (!(man & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline fp16_t fp32_to_fp16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (fp16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (fp16_t)(sign | 0x7C00u);  // rounds past 65504
    if (ax < 0x38800000u) {                                    // half subnormal or zero
        if (ax < 0x33000000u) return (fp16_t)sign;             // below half of the smallest subnormal
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126 - e;  // 14..24
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (fp16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (fp16_t)(sign | r);
}

inline void fp16_to_fp32_row(const fp16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = fp16_to_fp32(src[i]);
}

inline void fp32_to_fp16_row(const float* src, fp16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = fp32_to_fp16(src[i]);
}
