// fb_tanhf.h -- tanhf bit-identical to glibc 2.35.
//
// The quantile gradient of the reference CPU engine calls the host libm's
// tanhf (Objective::quantile_gradient, src/training/objective.rs:1142-1160:
// x.tanh() in f32). glibc up to 2.40 computes tanhf by the fdlibm method
// (Sun Microsystems, s_tanhf.c / s_expm1f.c, float versions by Ian Lance
// Taylor), which this file restates:
//
//   tanh(x) = sign(x) * (1 - 2 / (expm1(2|x|) + 2))   for 1 <= |x| < 22,
//           = sign(x) * -t / (t + 2), t = expm1(-2|x|) for 2^-55 <= |x| < 1,
//           = x (1 + x) below 2^-55, +-(1 - tiny) from 22 up;
//
//   expm1(x): reduce x = k ln2 + r with ln2 split into a 24-bit head
//   (0x3f317180) and a tail (0x3717f7d1), |r| <= ln2 / 2, then the rational
//   approximation of fdlibm with the scaled coefficients Q1..Q5 of
//   6/r (1 + 2 (1 / (e^r - 1) - 1 / r)) and the published reconstruction
//   2^k (e^r - 1) + (2^k - 1) for each range of k.
//
// Every operation is a single rounded float operation (no contraction: the
// including translation units build with -ffp-contract=off), so the host and
// device compiles give the same bits. Checked against glibc 2.35's tanhf on
// every one of the 2^32 float inputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fbh {

__host__ __device__ inline float tanh_bits_float(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint32_t tanh_float_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

__host__ __device__ inline float fb_expm1f(float x) {
    constexpr float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
    constexpr float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    constexpr float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    constexpr float invln2 = 1.4426950216e+00f;  // 0x3fb8aa3b
    constexpr float o_threshold = 8.8721679688e+01f;
    constexpr float Q1 = -3.3333335072e-02f;     // 0xbd088889
    constexpr float Q2 = 1.5873016091e-03f;      // 0x3ad00d01
    constexpr float Q3 = -7.9365076090e-05f;     // 0xb8a670cd
    constexpr float Q4 = 4.0082177293e-06f;      // 0x36867e54
    constexpr float Q5 = -2.0109921195e-07f;     // 0xb457edbb
    uint32_t hx = tanh_float_bits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    float y;
    if (hx >= 0x4195b844u) {       // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {   // |x| >= 88.72...
            if (hx > 0x7f800000u) return x + x;  // NaN
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;  // x < -27 ln2
    }
    float hi, lo, c = 0.0f, t;
    int32_t k;
    if (hx > 0x3eb17218u) {        // |x| > ln2 / 2
        if (hx < 0x3f851592u) {    // and |x| < 3 ln2 / 2
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;   // exact
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) { // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return one + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {       // exp(x) - 1 ~ exp(x)
        y = one - (e - x);
        if (k == 128)
            y = y * 2.0f * 0x1p127f;
        else
            y = tanh_bits_float(tanh_float_bits(y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = tanh_bits_float(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
        y = tanh_bits_float(tanh_float_bits(y) + ((uint32_t)k << 23));
    } else {
        t = tanh_bits_float((uint32_t)(0x7f - k) << 23);       // 2^-k
        y = x - (e + t);
        y += one;
        y = tanh_bits_float(tanh_float_bits(y) + ((uint32_t)k << 23));
    }
    return y;
}

__host__ __device__ inline float fb_tanhf(float x) {
    constexpr float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    const uint32_t jx = tanh_float_bits(x);
    const uint32_t ix = jx & 0x7fffffffu;
    const bool neg = (jx >> 31) != 0;
    if (ix >= 0x7f800000u) return neg ? one / x - one : one / x + one;  // +-inf, NaN
    float z;
    if (ix < 0x41b00000u) {        // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (one + x);  // |x| < 2^-55
        const float ax = tanh_bits_float(ix);
        if (ix >= 0x3f800000u) {   // |x| >= 1
            const float t = fb_expm1f(two * ax);
            z = one - two / (t + two);
        } else {
            const float t = fb_expm1f(-two * ax);
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return neg ? -z : z;
}

}  // namespace fbh
