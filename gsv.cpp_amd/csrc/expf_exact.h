// expf with the results of glibc's expf on x86-64 (the libm the reference's ggml-cpu build and the
// oracle call in flash attention's online softmax), bit for bit, for the device and the host.
//
// Method (published in ARM's optimized-routines and used by glibc >= 2.27): with N = 32,
//   z = x * N / ln2, k = round(z) (by adding and removing 1.5 * 2^52), r = z - k in [-1/2, 1/2];
//   exp(x) = 2^(k/N) * 2^(r/N) ~= s * (C0 r^3 + C1 r^2 + C2 r + 1), s = 2^(k/N) from a 32-entry
//   table of 2^(i/N) whose exponent field takes k / N;
// all in double, rounded to float once at the end. glibc's x86-64 build runs the variant compiled
// with FMA (selected at run time on FMA hardware), in which z + shift, z - k and the polynomial are
// fused multiply-adds; the fused steps are written out here. The table holds the bits of the
// double nearest 2^(i/32) minus i << 47 (computed from exact decimal arithmetic). Checked against
// the host's expf on every non-NaN float (tests/native/expf_check.cpp).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define GSVK_HD __host__ __device__
#else
#define GSVK_HD
#include <cmath>
#include <cstring>
#endif

// 2^(i/32) as double bits minus (i << 47), i < 32
#define GSVK_EXP2_TAB32                                                                          \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

namespace gsvk {

GSVK_HD inline uint32_t expf_bits32(float f) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, f);
#else
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
#endif
}
GSVK_HD inline uint64_t expf_bits64(double d) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint64_t, d);
#else
    uint64_t u;
    std::memcpy(&u, &d, 8);
    return u;
#endif
}
GSVK_HD inline double expf_from_bits64(uint64_t u) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, u);
#else
    double d;
    std::memcpy(&d, &u, 8);
    return d;
#endif
}

// tab: the 32 entries of GSVK_EXP2_TAB32 (the caller's copy: constant memory on the device)
GSVK_HD inline float expf_glibc(float x, const uint64_t * tab) {
    const uint32_t abstop = (expf_bits32(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                                    // |x| >= 88 or NaN
        if (expf_bits32(x) == 0xff800000u) return 0.0f;       // -inf
        if (abstop >= 0x7f8) return x + x;                    // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff();       // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                  // underflow
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double) x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = expf_bits64(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = expf_from_bits64(t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float) y;
}

}  // namespace gsvk
