// CPU check of the parallel exact running-sum method in
// ax-engine_amd/csrc/axs_exact_sum.h: a block of T "threads" × IT items per
// tile is simulated exactly as the HIP kernel runs it (per-thread transducers,
// exclusive prefix, per-item walk, first crossing handled by a plain f32 add),
// and every prefix must equal the sequential f32 running sum bit for bit.
// Built and run by tests/test_exact_sum.py.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cmath>
#include <vector>
#include <random>
#include <algorithm>
#include "axs_exact_sum.h"

using namespace axs;

static void block_scan(const std::vector<float>& x, std::vector<float>& out, int T, int IT) {
    size_t n = x.size();
    out.assign(n, 0.0f);
    float s = 0.0f;
    size_t k = 0;
    while (k < n) {
        Binade bd = binade_of(s);
        size_t tile = std::min<size_t>((size_t)T * IT, n - k);
        std::vector<Xd> tx(T, xd_identity());
        for (int t = 0; t < T; ++t)
            for (int j = 0; j < IT; ++j) {
                size_t i = k + (size_t)t * IT + j;
                if (i >= k + tile) break;
                tx[t] = xd_compose(tx[t], xd_of(term_of(x[i], bd.E)));
            }
        size_t first_cross = (size_t)-1;
        Xd pre = xd_identity();
        for (int t = 0; t < T; ++t) {
            uint32_t b0 = bd.A & 1u;
            uint64_t a = bd.A + (b0 ? pre.inc1 : pre.inc0);
            uint32_t par = b0 ? pre.par1 : pre.par0;
            for (int j = 0; j < IT; ++j) {
                size_t i = k + (size_t)t * IT + j;
                if (i >= k + tile) break;
                Term tm = term_of(x[i], bd.E);
                uint32_t c = par ? tm.c1 : tm.c0;
                if (a + c >= (1ull << 24)) {
                    if (i < first_cross) first_cross = i;
                    break;
                }
                a += c;
                par = (uint32_t)(a & 1u);
                out[i] = binade_value((uint32_t)a, bd.E);
            }
            pre = xd_compose(pre, tx[t]);
        }
        if (first_cross == (size_t)-1) {
            s = out[k + tile - 1];
            k += tile;
        } else {
            float prev = first_cross == k ? s : out[first_cross - 1];
            s = prev + x[first_cross];
            out[first_cross] = s;
            k = first_cross + 1;
        }
    }
}

static int check(const std::vector<float>& x, int T, int IT, const char* name) {
    std::vector<float> out;
    block_scan(x, out, T, IT);
    float s = 0.0f;
    for (size_t i = 0; i < x.size(); ++i) {
        s = s + x[i];
        if (memcmp(&s, &out[i], 4) != 0) {
            std::printf("FAIL %s at %zu: seq %.9g got %.9g\n", name, i, (double)s, (double)out[i]);
            return 1;
        }
    }
    return 0;
}

int main() {
    std::mt19937_64 g(12345);
    int fails = 0, cases = 0;
    std::normal_distribution<double> nd(0.0, 1.0);
    std::uniform_real_distribution<double> ud(0.0, 1.0);
    for (int rep = 0; rep < 60; ++rep) {
        size_t n = 1 + (g() % 20000);
        double sigma = 1.0 + 4.0 * ud(g);
        double inv = 0.5 + 2.0 * ud(g);
        std::vector<float> l(n);
        for (auto& v : l) v = (float)(nd(g) * sigma);
        if (rep % 3 == 0)  // bf16-like: coarse values, many exact repeats
            for (auto& v : l) { uint32_t b; memcpy(&b, &v, 4); b &= 0xFFFF0000u; memcpy(&v, &b, 4); }
        float m = *std::max_element(l.begin(), l.end());
        std::vector<float> p(n);
        for (size_t i = 0; i < n; ++i) p[i] = std::exp((l[i] - m) * (float)inv);
        // index order
        fails += check(p, 64, 4, "index"); ++cases;
        // sorted descending (the nucleus order)
        std::vector<float> ps = p;
        std::sort(ps.begin(), ps.end(), [](float a, float b) { return a > b; });
        fails += check(ps, 64, 4, "sorted"); ++cases;
        fails += check(ps, 256, 2, "sorted-256x2"); ++cases;
    }
    // crafted: exact half-ulp ties, powers of two, zeros, subnormals
    {
        std::vector<float> x;
        for (int i = 0; i < 5000; ++i) {
            int k = (int)(g() % 7);
            float v = 0.0f;
            if (k == 0) v = std::ldexp(1.0f, -(int)(g() % 30));
            else if (k == 1) v = std::ldexp(3.0f, -(int)(g() % 40) - 1);
            else if (k == 2) v = 0.0f;
            else if (k == 3) v = std::ldexp(1.0f, -140 - (int)(g() % 9));
            else if (k == 4) v = (float)ud(g);
            else if (k == 5) v = std::ldexp((float)(1 + 2 * (g() % 1000)), -24 - (int)(g() % 5));
            else v = 1.0f;
            x.push_back(v);
        }
        fails += check(x, 64, 4, "crafted"); ++cases;
        std::sort(x.begin(), x.end(), [](float a, float b) { return a > b; });
        fails += check(x, 64, 4, "crafted-sorted"); ++cases;
        std::vector<float> ones(100000, 1.0f);
        fails += check(ones, 64, 4, "ones"); ++cases;
        std::vector<float> tiny(3000, std::ldexp(1.0f, -149));
        fails += check(tiny, 64, 4, "denorm"); ++cases;
    }
    std::printf("%d cases, %d failures\n", cases, fails);
    return fails ? 1 : 0;
}
