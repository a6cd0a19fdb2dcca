// Fixed-point quantisation of one f32 gradient under a power-of-two scale
// (GradQuantizer::to_fixed, src/types.rs:367-385): round half away from zero
// of v * 2^l, saturated to int64, NaN to 0. The double formula
// sat_i64(round((double)v * 2^l)) is exact in double for the scales the
// quantizer makes (2^l, |l| <= 1000), so this integer form gives the same
// value for every float: v = m * 2^e with an integer mantissa m < 2^24,
// hence v * 2^l = m * 2^(e + l), a shift of m.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define FBQ_FN __host__ __device__ __forceinline__
#else
#define FBQ_FN inline
#endif

namespace fbh {

// The l of a scale 2^l (the biased exponent of a normal double minus 1023).
FBQ_FN int pow2_exponent(double scale) {
    uint64_t b;
    memcpy(&b, &scale, 8);
    return (int)((b >> 52) & 0x7FF) - 1023;
}

FBQ_FN int64_t quantize_pow2(float v, int l) {
    uint32_t b;
    memcpy(&b, &v, 4);
    const uint32_t E = (b >> 23) & 0xFFu, F = b & 0x7FFFFFu;
    const bool neg = (b >> 31) != 0;
    if (E == 0xFFu) {  // NaN -> 0, +-inf saturate
        if (F) return 0;
        return neg ? (int64_t)0x8000000000000000ull : (int64_t)0x7FFFFFFFFFFFFFFFll;
    }
    const uint32_t m = E ? (F | 0x800000u) : F;  // |v| = m * 2^s
    if (m == 0) return 0;                        // +-0
    const int s = (E ? (int)E - 150 : -149) + l;
    uint64_t mag;
    if (s >= 0) {
        // m < 2^24: below 2^63 for s <= 39; beyond, saturated once m * 2^s
        // reaches 2^63.
        if (s > 39 && (s >= 63 || (uint64_t)m >= (1ull << (63 - s))))
            return neg ? (int64_t)0x8000000000000000ull : (int64_t)0x7FFFFFFFFFFFFFFFll;
        mag = (uint64_t)m << s;
    } else if (s <= -25) {
        mag = 0;  // m * 2^s < 2^-1: rounds to zero
    } else {
        const int r = -s;  // 1..24; m + 2^(r-1) < 2^25
        mag = (uint64_t)((m + (1u << (r - 1))) >> r);
    }
    return neg ? -(int64_t)mag : (int64_t)mag;
}

}  // namespace fbh
