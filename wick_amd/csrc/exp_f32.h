// exp_f32.h -- f32 exp with the results of wick's f32::exp on x86-64 Linux.
//
// Rust's f32::exp (the softmax of Sampler::sample, /root/reference/src/sampler.rs:97)
// is a call to the C library's expf.  glibc (2.28 and later; this image has
// 2.35) implements it by the published table method of ARM's
// optimized-routines, built for x86-64 CPUs with FMA as the variant the
// library selects on them: with N = 32,
//   z = x * N / ln 2 in double, k = round(z) (ties to even, by adding and
//   subtracting 1.5 * 2^52), r = z - k as one fused multiply-add,
//   exp(x) = 2^(k/N) * 2^(r/N), 2^(r/N) ~ 1 + c2 r + c1 r^2 + c0 r^3,
//   2^(k/N) from a 32-entry table of 2^(i/32) whose exponent field takes
//   k / N directly,
// rounded once to f32 at the end.  The table entries are 2^(i/32) rounded to
// double, each less i << 47 so that adding k << 47 sets the exponent.  The
// same arithmetic in the same order gives the same bits: an exhaustive check
// over all 2^32 inputs against the host's expf finds no difference
// (tests/test_exp_f32.py).  glibc's build for CPUs without FMA (r as a
// rounded product then a subtraction) differs from this in 2 of the 2^32
// inputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wick {

__host__ __device__ inline float exp_f32(float x) {
#pragma clang fp contract(off)
    constexpr double N = 32.0;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * N;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / (N * N * N), kC1 = 0x1.ebfce50fac4f3p-3 / (N * N),
                     kC2 = 0x1.62e42ff0c52d6p-1 / N;
    constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
        0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
        0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
        0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
        0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
        0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
        0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
        0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 (the top 12 bits of 88.0f), or NaN / inf
        if (ux == 0xff800000u) return 0.0f;        // -inf
        if (abstop >= 0x7f8u) return x + x;        // NaN, +inf
        if (x > 0x1.62e42ep6f) return __builtin_inff();  // above log(2^128)
        if (x < -0x1.9fe368p6f) return 0.0f;       // below log(2^-150)
    }
    const double xd = (double)x;
    const double z = kInvLn2N * xd;
    double kd = z + kShift;
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, kTab[ki % 32] + (ki << 47));
    const double p = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    return (float)(y * s);
}

}  // namespace wick
