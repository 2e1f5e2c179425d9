// expf_glibc.h — exp(x) for f32 with the results of glibc's expf on x86-64.
//
// The reference evaluates SiLU and the sigmoid router with Rust's f32::exp
// (crates/peregrine-model/src/math.rs:108-111, router.rs:52-170), which on
// Linux calls glibc's expf. glibc (2.28 and later) implements expf with the
// published ARM optimized-routines method (Szabolcs Nagy, "expf", 2017): with
// N = 32, k = round(x * N / ln 2), r = x * N / ln 2 - k in [-1/2, 1/2],
//     exp(x) = 2^(k/N) * 2^(r/N),  2^(r/N) ~= C0 r^3 + C1 r^2 + C2 r + 1,
// all in double, then one rounding to f32. 2^(k/N) is the table entry
// T[k % N] with k/N added to its exponent field; the rounding of x*N/ln2 to
// an integer uses the 1.5*2^52 shift. On a CPU with FMA, glibc selects a
// build of this code in which every a*b+c is one fused multiply-add; that is
// the form below (explicit fma, so it holds under -ffp-contract=off). A sweep
// over all 2^32 f32 inputs against the host's glibc expf is part of the CPU
// tests (tests/test_expf.py): zero differences.
//
// The same source compiles for the host (g++) and the device (hipcc).
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define PHIP_HD __host__ __device__
#else
#define PHIP_HD
#endif

namespace phip_expf {

// T[i] = bits(2^(i/32) rounded to the nearest double) - (i << 47): adding
// k << 47 to T[k % 32] then yields the bits of 2^(k/32).
constexpr uint64_t T[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
constexpr double INV_LN2_N = 0x1.71547652b82fep+0 * 32;   // N / ln 2
constexpr double SHIFT = 0x1.8p+52;                         // rounds to an integer in the low bits
// the polynomial of 2^(r/N) with the powers of N folded in (exact: N = 2^5)
constexpr double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
constexpr double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
constexpr double C2 = 0x1.62e42ff0c52d6p-1 / 32;

PHIP_HD inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
PHIP_HD inline uint64_t f64_bits(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
PHIP_HD inline double f64_from(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}

}  // namespace phip_expf

PHIP_HD inline float expf_glibc(float x) {
    using namespace phip_expf;
    const uint32_t abstop = (f32_bits(x) >> 20) & 0x7ff;
    if (abstop >= (f32_bits(88.0f) >> 20)) {   // |x| >= 88, inf or NaN
        if (f32_bits(x) == f32_bits(-INFINITY)) return 0.0f;
        if (abstop >= (f32_bits(INFINITY) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;   // above log(2^128)
        if (x < -0x1.9fe368p6f) return 0.0f;      // below log(2^-150)
    }
    const double xd = (double)x;
    double kd = fma(INV_LN2_N, xd, SHIFT);
    const uint64_t ki = f64_bits(kd);
    kd -= SHIFT;
    const double r = fma(INV_LN2_N, xd, -kd);
    const double s = f64_from(T[ki % 32] + (ki << 47));
    const double z = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}
