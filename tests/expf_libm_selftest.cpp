// CPU check of axs::expf_libm (ax-engine_amd/csrc/axs_expf.h), the device's
// f32 exp: over every one of the 2^32 f32 inputs its result must be bit-
// identical to the host libm's expf (what the reference's f32::exp calls on
// Linux), NaN results compared as NaN.  It also checks that expf is
// monotone non-decreasing over x <= 0, which the sampler's min-p edge search
// (the smallest x with exp(x) >= min_p) assumes.  Built and run by
// tests/test_expf_libm.py; prints "0 mismatches, 0 inversions" when clean.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "axs_expf.h"

static float as_f(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static uint32_t as_u(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

int main(int argc, char** argv) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    std::vector<uint64_t> bad(nt, 0), inv(nt, 0);
    std::vector<std::thread> th;
    for (unsigned id = 0; id < nt; ++id) {
        th.emplace_back([&, id] {
            const uint64_t n = 1ull << 32, per = (n + nt - 1) / nt;
            const uint64_t lo = id * per, hi = std::min<uint64_t>(n, lo + per);
            for (uint64_t b = lo; b < hi; ++b) {
                const float x = as_f((uint32_t)b);
                const float want = expf(x), got = axs::expf_libm(x);
                const bool same = (want != want) ? (got != got) : as_u(want) == as_u(got);
                if (!same) {
                    if (bad[id] < 4) std::printf("mismatch x=%a libm=%a restated=%a\n", x, want, got);
                    ++bad[id];
                }
            }
            // monotone over x <= 0: walk the negative floats from -0 down to
            // -inf, i.e. bit patterns 0x80000000 .. 0xFF800000 in order.
            const uint64_t m0 = 0x80000000ull, m1 = 0xFF800000ull, mp = (m1 - m0 + nt - 1) / nt;
            const uint64_t a = m0 + id * mp, e = std::min<uint64_t>(m1, a + mp);
            for (uint64_t b = a; b < e; ++b) {
                const float hi_x = as_f((uint32_t)b), lo_x = as_f((uint32_t)(b + 1));  // lo_x < hi_x
                if (axs::expf_libm(lo_x) > axs::expf_libm(hi_x)) {
                    if (inv[id] < 4) std::printf("inversion at %a\n", lo_x);
                    ++inv[id];
                }
            }
        });
    }
    for (auto& t : th) t.join();
    uint64_t nb = 0, ni = 0;
    for (unsigned i = 0; i < nt; ++i) {
        nb += bad[i];
        ni += inv[i];
    }
    std::printf("%llu mismatches, %llu inversions\n", (unsigned long long)nb, (unsigned long long)ni);
    return (nb || ni) ? 1 : 0;
}
