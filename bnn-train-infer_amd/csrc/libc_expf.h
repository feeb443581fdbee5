/*
 * expf with the results of the host C library's expf (glibc 2.35 on x86-64, whose
 * expf runs the FMA build of the table-driven method of ARM's optimized-routines):
 *
 *   k = round(x * 32/ln2) (by adding 1.5*2^52),  r = x * 32/ln2 - k,
 *   2^(k/32) = T[k mod 32] with k's high bits added into the exponent field,
 *   exp(x) ~= 2^(k/32) * (1 + c2 r + c1 r^2 + c0 r^3), in double, fused multiply-
 *   adds where that build has them, rounded once to float;
 *   |x| >= 88: -inf -> 0, NaN/+inf -> x + x, overflow -> +inf, underflow -> +0.
 *
 * T[i] is 2^(i/32) correctly rounded to double, minus i << 47 (so that adding
 * k << 47 restores it and scales by 2^(k div 32)).  The polynomial coefficients are
 * those of the published method (2^(r/32) in r, scaled by powers of 1/32).
 *
 * One source for the device (the backend's fused SiLU pre-operation, the engine's
 * kernels) and for the test-side host check that compares it with the C library on
 * every float.
 * Plain C: define BNNE_EXPF_QUALIFIER for device compilation.
 */
#ifndef BNNE_LIBC_EXPF_H
#define BNNE_LIBC_EXPF_H

#include <stdint.h>
#include <string.h>

#ifndef BNNE_EXPF_QUALIFIER
#define BNNE_EXPF_QUALIFIER static inline
#endif

#define BNNE_EXP2_TABLE                                                                            \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

BNNE_EXPF_QUALIFIER float bnne_expf_libc(float x, const uint64_t* table) {
    uint32_t ux;
    memcpy(&ux, &x, sizeof ux);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) { /* |x| >= 88, or not finite */
        if (ux == 0xff800000u)
            return 0.0f;
        if (abstop >= 0x7f8u)
            return x + x;
        if (x > 0x1.62e42ep6f) {
            const uint32_t inf = 0x7f800000u;
            float r;
            memcpy(&r, &inf, sizeof r);
            return r;
        }
        if (x < -0x1.9fe368p6f)
            return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, sizeof ki);
    kd = kd - shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t t = table[ki % 32u] + (ki << 47);
    double s;
    memcpy(&s, &t, sizeof s);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

#endif
