// fb_expf.h -- expf and the logistic sigmoid, bit-identical to glibc.
//
// The logistic gradient of the reference CPU engine calls the host libm's
// expf (src/training/objective.rs:37-39: 1 / (1 + exp(-x)) in f32). glibc
// (2.28 and later) computes expf by the table-driven method of Szabolcs Nagy
// (ARM optimized-routines): with N = 32, x * N / ln2 = k + r, |r| <= 1/2,
// 2^(k/N) = 2^(k>>5) * T[k & 31] and 2^(r/N) ~ 1 + C2 r + C1 r^2 + C0 r^3,
// all in double, rounded once to float. This file restates that method:
//   T[i]  = 2^(i/32) rounded to nearest double, stored minus i << 47 so that
//           adding k << 47 to the bits rebuilds 2^(k/32);
//   C     = the published cubic 0x1.c6af84b912394p-5, 0x1.ebfce50fac4f3p-3,
//           0x1.62e42ff0c52d6p-1 scaled by N^-3, N^-2, N^-1;
//   k     = round(x * N / ln2) through the 1.5 * 2^52 shift.
// The multiply-adds are fused (fma) as in glibc's FMA build. Checked against
// glibc 2.35 on every one of the 2^32 float inputs: expf bit-identical, and
// 1 / (1 + expf(-x)) bit-identical also for the unfused build.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fbh {

__host__ __device__ inline uint64_t exp_tab(uint32_t i) {
    constexpr uint64_t T[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull,
    0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull,
    0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull,
    0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull,
    0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull,
    0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull
    };
    return T[i];
}

__host__ __device__ inline float fb_expf(float x) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 or x is NaN
        if (ux == 0xff800000u) return 0.0f;               // -inf
        if (abstop >= 0x7f8u) return x + x;               // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff();   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
    }
    constexpr double INVLN2N = 0x1.71547652b82fep+0 * 32.0;
    constexpr double SHIFT = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(INVLN2N, xd, SHIFT);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd = kd - SHIFT;
    const double r = __builtin_fma(INVLN2N, xd, -kd);
    const double s = __builtin_bit_cast(double, exp_tab((uint32_t)(ki & 31u)) + (ki << 47));
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// sigmoid (src/training/objective.rs:37-39) with the host's f32 operations.
__host__ __device__ inline float fb_sigmoid(float m) { return 1.0f / (1.0f + fb_expf(-m)); }

}  // namespace fbh
