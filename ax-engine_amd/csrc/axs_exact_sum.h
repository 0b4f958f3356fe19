// axs_exact_sum.h — reproducing a sequential f32 running sum in parallel.
//
// The reference accumulates probabilities one by one in f32
// (`cumsum += p`, `iter().sum()`: crates/ax-engine-mlx/src/sampling.rs:258,278,
// 297,304,935-941), and with ~1e5 terms that running sum drifts from the exact
// sum by up to ~1e-3 relative.  Token decisions (nucleus edge, draw point)
// depend on those rounded values, so the sampler reproduces the running sum
// bit for bit.
//
// Method.  While the running sum s stays inside one binade [2^e, 2^(e+1))
// (or below 2^-125, where the spacing is 2^-149 throughout), every f32 value
// there is an integer multiple of U = ulp(s), and fl(s + x) = s + c*U with
// c = round(x / U) — except when x / U is exactly n + 1/2, where round-half-
// to-even makes c depend on the parity of s / U.  So each term is a two-state
// transducer (parity in → increment, parity out).  Transducers compose
// associatively, which turns the running sum into a parallel prefix scan.  A
// term whose add could leave the binade (s/U + c >= 2^24) is done as an
// ordinary f32 add, after which the scan restarts in the new binade.
//
// The helpers here are __host__ __device__ so the same code is unit-tested
// on the CPU against a plain sequential loop.
#pragma once

#include <stdint.h>
#include <string.h>
#include <math.h>

#ifdef __HIPCC__
#define AXS_HD __host__ __device__ __forceinline__
#else
#define AXS_HD static inline
#endif

namespace axs {

// Binade parameters of a non-negative running sum s: U = 2^E, A = s / U
// (an exact integer < 2^24).
struct Binade {
    int32_t E;   // log2 of the spacing
    uint32_t A;  // s / 2^E
};

AXS_HD uint32_t f32_bits(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return b;
}

AXS_HD float bits_f32(uint32_t b) {
    float x;
    memcpy(&x, &b, 4);
    return x;
}

AXS_HD Binade binade_of(float s) {
    // s >= 0 and finite.  Biased exponent 0 (subnormal/zero) and 1 (the first
    // normal binade) share the spacing 2^-149.
    uint32_t b = f32_bits(s);
    uint32_t ex = (b >> 23) & 0xFFu;
    Binade r;
    if (ex <= 1u) {
        r.E = -149;
        r.A = b & 0x00FFFFFFu;  // for ex==1 this is (1<<23)|mantissa
    } else {
        r.E = (int32_t)ex - 127 - 23;
        r.A = (b & 0x007FFFFFu) | 0x00800000u;
    }
    return r;
}

// s = A * 2^E, exact for A < 2^24: inside a normal binade (A >= 2^23) or in
// the lowest one (E = -149) it is the bit pattern ((E + 149) << 23) + A.
AXS_HD float binade_value(uint32_t A, int32_t E) {
    if (E == -149 || A >= 0x00800000u) return bits_f32(((uint32_t)(E + 149) << 23) + A);
    return (float)ldexp((double)A, E);
}

// Increment of one term x (>= 0, finite) in units of U = 2^E:
// c0 for an even running sum, c1 for an odd one; saturated at 2^25 (a term
// that large always leaves the binade).
struct Term {
    uint32_t c0, c1;
};

AXS_HD Term term_of(float x, int32_t E) {
    // x = M * 2^e2 with M its 24-bit significand; q = x / 2^E = M * 2^(e2 - E),
    // split into integer part n and remainder r of sh bits, all in integers
    const uint32_t b = f32_bits(x);
    const uint32_t be = b >> 23;  // x >= 0: no sign bit
    const uint32_t M = be ? ((b & 0x007FFFFFu) | 0x00800000u) : (b & 0x007FFFFFu);
    const int32_t s = (be ? (int32_t)be - 150 : -149) - E;
    Term t;
    if (s >= 0) {
        const uint64_t q = (uint64_t)M << (s < 40 ? s : 40);
        t.c0 = t.c1 = q >= 33554432ull ? 33554432u : (uint32_t)q;  // saturated at 2^25
        return t;
    }
    const uint32_t sh = (uint32_t)(-s);
    if (sh >= 26u) {  // q < 2^24 / 2^26: rounds to 0
        t.c0 = t.c1 = 0u;
        return t;
    }
    const uint32_t ni = M >> sh;
    const uint32_t r = M & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (r > half) {
        t.c0 = t.c1 = ni + 1u;
    } else if (r < half) {
        t.c0 = t.c1 = ni;
    } else {  // exact tie: round half to even on (s/U + n + 1/2)
        t.c0 = ni + (ni & 1u);
        t.c1 = ni + ((ni + 1u) & 1u);
    }
    return t;
}

// Composition of terms: starting parity b in {0,1} → (total increment,
// ending parity).
struct Xd {
    uint64_t inc0, inc1;
    uint32_t par0, par1;
};

AXS_HD Xd xd_identity() {
    Xd r;
    r.inc0 = 0; r.inc1 = 0; r.par0 = 0; r.par1 = 1;
    return r;
}

AXS_HD Xd xd_of(Term t) {
    Xd r;
    r.inc0 = t.c0;
    r.par0 = t.c0 & 1u;
    r.inc1 = t.c1;
    r.par1 = (1u + t.c1) & 1u;
    return r;
}

// a then b
AXS_HD Xd xd_compose(Xd a, Xd b) {
    Xd r;
    r.inc0 = a.inc0 + (a.par0 ? b.inc1 : b.inc0);
    r.par0 = a.par0 ? b.par1 : b.par0;
    r.inc1 = a.inc1 + (a.par1 ? b.inc1 : b.inc0);
    r.par1 = a.par1 ? b.par1 : b.par0;
    return r;
}

// Sequential reference: the f32 running sum, one add at a time.
AXS_HD float seq_add(float s, float x) { return s + x; }

}  // namespace axs
