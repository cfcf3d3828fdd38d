// libm_expf.h - expf with glibc's results, bit for bit, on the host and the device.
//
// The reference's sample_temperature (utils.c:158-180) weighs each token with libm's expf,
// and a draw compares against running sums of those weights, so the device must produce the
// very same floats. glibc (2.27 and later) implements expf with Arm's optimized-routines
// method (Szabolcs Nagy, 2017, MIT licensed): x = (k + r) ln2 / 32 with integer k and
// |r| <= 1/2, exp(x) = 2^(k/32) 2^(r/32), 2^(k/32) from a 32-entry table of 2^(i/32) with the
// exponent added in the integer domain, 2^(r/32) from a cubic, all in double, one final
// rounding to float. On x86-64 with FMA glibc runs the build of it compiled with -mfma, whose
// contracted forms are written out below; this restatement agrees with that glibc expf on
// every float in [-104, 0] (the range sample_temperature feeds it: (l - max) / T <= 0), and
// follows the same special cases elsewhere.
#pragma once

#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#define SPH_HD __host__ __device__
#else
#define SPH_HD
#endif

namespace sapphire {

SPH_HD inline double libm_as_double(uint64_t u) {
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
}

SPH_HD inline uint64_t libm_as_u64(double d) {
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
}

SPH_HD inline float libm_expf(float x) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    // tab[i] = bits of 2^(i/32) (rounded to nearest double) minus i << 47, so that adding
    // k << 47 for k = 32 q + i gives the bits of 2^q 2^(i/32)
    constexpr uint64_t tab[32] = {
        0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
        0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
        0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
        0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
        0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
        0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
        0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
        0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
    };
    constexpr double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;   // 32 / ln 2
    constexpr double shift = 0x1.8p+52;                        // rounds to an integer in the low bits
    // 2^(r/32) ~= c0 r^3 + c1 r^2 + c2 r + 1 (minimax coefficients of the published method)
    constexpr double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    memcpy(&ux, &x, sizeof ux);
    if ((ux & 0x7fffffffu) >= 0x42b00000u) {      // |x| >= 88, infinities, NaN
        if (ux == 0xff800000u) return 0.0f;       // -inf
        if ((ux & 0x7fffffffu) >= 0x7f800000u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = libm_as_u64(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const double s = libm_as_double(tab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

}  // namespace sapphire
