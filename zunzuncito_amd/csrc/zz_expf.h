// zz_expf.h -- expf with the bits of glibc's (x86-64, glibc 2.27 and later).
//
// lfm25.c:654 and ling.c:731 route a token by 1/(1+expf(-v)): one last-bit
// difference in expf can move a selection score across another expert's, and
// glibc's expf is not correctly rounded on every input (it differs from the
// correctly rounded exp on ~1.6e5 floats in |x| < 40). So the device evaluates the
// algorithm glibc uses for expf since 2.27, the one published with ARM's
// optimized-routines (Szabolcs Nagy, 2017, MIT / Apache-2.0):
//   with N = 32, x*N/ln2 = k + r, |r| <= 1/2, k an integer (rounded to nearest by
//   adding 1.5*2^52 and reading the low mantissa bits);
//   exp(x) = 2^(k/N) * 2^(r/N) ~= s * (C0 r^3 + C1 r^2 + C2 r + 1),
// where s = 2^(k/N) is formed from a table of 2^(i/N), i < N (correctly rounded
// doubles stored minus i << 47, so that adding k << 47 scales by 2^(k/N)), and
// C0..C2 are the algorithm's published minimax coefficients for 2^(r/N). The whole
// evaluation is in double, rounded to float once. On CPUs with FMA, x86-64 glibc
// runs a build of it compiled with -mfma, where gcc fuses x*N/ln2 into both of its
// uses (the shift add and r) and the polynomial's multiply-adds; the same fmas are
// written here. The table is 2^(i/32) rounded to double (derivable from the
// mathematics); the host test compares this function with the host's expf on all
// 2^32 inputs and the GPU test compares the device's results with it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// 2^(i/32) as double bits, minus i << 47
static constexpr uint64_t zz_exp2_tab32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// TAB: the table's entry i (the table itself, or a copy of it nearer the caller)
template <typename TAB>
__host__ __device__ inline float zz_expf_tab(float x, TAB tab) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                       // |x| >= 88 (the top 12 bits of 88.0f), or NaN
        if (ux == 0xff800000u) return 0.0f;       // -inf
        if (abstop >= 0x7f8u) return x + x;       // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();   // above log(2^128): overflow
        if (x < -0x1.9fe368p6f) return 0.0f;      // below log(2^-150): underflow
    }
    const double n_ln2 = 0x1.71547652b82fep+0 * 32;       // N / ln 2
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = fma(n_ln2, xd, shift);            // k in the low bits of kd
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = fma(n_ln2, xd, -kd);
    const uint64_t t = tab((int)(ki % 32)) + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

__host__ __device__ inline float zz_expf(float x) {
    return zz_expf_tab(x, [](int i) { return zz_exp2_tab32[i]; });
}
