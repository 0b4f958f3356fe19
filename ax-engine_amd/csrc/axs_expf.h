// axs_expf.h — an f32 exp whose every result equals the host libm's expf.
//
// The reference computes probabilities with Rust's f32::exp
// (crates/ax-engine-mlx/src/sampling.rs:248-251,274-277,690-695), which on
// Linux is the C library's expf.  Since glibc 2.27 that is the table-driven
// method of ARM's optimized-routines (Szabolcs Nagy, 2017; glibc
// sysdeps/ieee754/flt-32/e_expf.c), and on x86-64 hosts with FMA glibc
// selects its FMA-compiled variant.  The method, with N = 32:
//
//   z  = x * (N / ln 2)                 (double)
//   k  = round-to-nearest-even(z)
//   r  = fma(N / ln 2, x, -k)           (the FMA build fuses the reduction)
//   s  = 2^(k / N) = bits(T[k mod N] + (k << 47)),
//        T[i] = bits(2^(i/N) rounded to double) - (i << 47)
//   exp(x) ~= s * (C0 r^3 + C1 r^2 + C2 r + 1), evaluated as
//        fma(fma(C0, r, C1), r*r, fma(C2, r, 1)) * s, then rounded to f32.
//
// C0..C2 are the method's published minimax coefficients of 2^(r/N); T is
// computed here from 2^(i/32) (60-digit decimal arithmetic, rounded to
// nearest double).  The restatement is compared with the host's expf over
// all 2^32 inputs on the CPU (tests/test_expf_libm.py, every result bit-
// identical), which also checks that it is monotone on the inputs the
// sampler feeds it (x <= 0), a property the min-p edge search relies on.
//
// Outside the reduction's range: x < ln(2^-150) (and -inf) gives 0,
// x > ln(2^128) gives +inf, NaN gives NaN — glibc's special cases.
#pragma once

#include <stdint.h>
#include <string.h>
#include <math.h>

#ifdef __HIPCC__
#define AXS_EXPF_HD __host__ __device__ __forceinline__
#define AXS_EXPF_TABLE __constant__
#else
#define AXS_EXPF_HD static inline
#define AXS_EXPF_TABLE
#endif

namespace axs {

AXS_EXPF_TABLE static const uint64_t kExp2Tab32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

AXS_EXPF_HD float expf_libm(float x) {
    if (!(x >= -0x1.9fe368p6f)) return x != x ? x + x : 0.0f;  // NaN; below ln 2^-150, -inf
    if (x > 0x1.62e42ep6f) return INFINITY;                     // above ln 2^128, +inf
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = kInvLn2N * xd;
    const double kd = rint(z);
    const int64_t ki = (int64_t)kd;
    const double r = fma(kInvLn2N, xd, -kd);
    const uint64_t t = kExp2Tab32[ki & 31] + ((uint64_t)ki << 47);
    double s;
    memcpy(&s, &t, sizeof(s));
    const double zc = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(zc, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace axs
