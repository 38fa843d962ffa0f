// CPU check of mimg::quant_rne (mimir-model_amd/csrc/quant_rne.hpp, the
// rounding the GPU quantizer kernels use) against an exact integer
// evaluation of RoundToEven(127*x/amax). Built and run by
// tests/test_quant_rne.py. Prints the number of mismatches and exits 1 if
// there are any.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>

#include "../mimir-model_amd/csrc/quant_rne.hpp"

// Exact RoundToEven(127*x/amax) with 128-bit integers, |x| <= amax, amax > 0.
static int exact_rne(float x, float amax) {
    int ex, ea;
    const double fx = std::frexp((double)x, &ex), fa = std::frexp((double)amax, &ea);
    const int64_t mx = (int64_t)std::ldexp(fx, 53), ma = (int64_t)std::ldexp(fa, 53);  // exact
    const bool neg = mx < 0;
    __int128 num = (__int128)127 * (neg ? -mx : mx), den = ma;
    const int s = ex - ea;  // q* = num * 2^s / den
    if (s >= 0) {
        num <<= s;  // |q*| <= 127 keeps this small
    } else {
        if (-s > 60) return 0;  // |q*| < 2^-50: rounds to 0
        den <<= -s;
    }
    __int128 q = num / den, r = num - q * den;
    if (2 * r > den || (2 * r == den && (q & 1))) q++;
    return neg ? -(int)q : (int)q;
}

int main(int argc, char** argv) {
    const long n = argc > 1 ? atol(argv[1]) : 2000000;
    std::mt19937_64 rng(12345);
    std::uniform_real_distribution<double> u(-1.0, 1.0);
    std::uniform_int_distribution<int> ee(-149, 60), nn(-127, 126);
    long bad = 0, checked = 0, ties = 0;
    auto check = [&](float x, float amax) {
        if (!(std::fabs(x) <= amax) || !(amax > 0)) return;
        const float inv = 1.0f / amax;
        const int got = mimg::quant_rne(x, amax, inv), want = exact_rne(x, amax);
        int fq;
        if (mimg::quant_rne_fast(x, amax, inv, fq) && fq != want) {
            if (bad < 10) printf("fast path: x=%a amax=%a got %d want %d\n", x, amax, fq, want);
            bad++;
        }
        checked++;
        if (got != want) {
            if (bad < 10) printf("x=%a amax=%a got %d want %d\n", x, amax, got, want);
            bad++;
        }
    };
    for (long i = 0; i < n; i++) {
        // random magnitudes over the whole float range up to 2^60
        const float amax = (float)std::ldexp(0.5 + 0.5 * std::fabs(u(rng)), ee(rng));
        check((float)(u(rng) * amax), amax);
        check(amax, amax);
        // exact ties: amax = 127*2^e, x = (k + 1/2) * 2^e, and their neighbours
        const int e = ee(rng) % 50;
        const float a2 = (float)std::ldexp(127.0, e);
        const float xt = (float)std::ldexp(nn(rng) + 0.5, e);
        check(xt, a2);
        check(std::nextafter(xt, INFINITY), a2);
        check(std::nextafter(xt, -INFINITY), a2);
        ties++;
        // near-ties for a general amax: x close to (k+1/2)*amax/127
        const float a3 = (float)std::ldexp(0.5 + 0.5 * std::fabs(u(rng)), ee(rng));
        const float x3 = (float)((nn(rng) + 0.5) * (double)a3 / 127.0);
        check(x3, a3);
        check(std::nextafter(x3, INFINITY), a3);
        check(std::nextafter(x3, -INFINITY), a3);
    }
    printf("checked %ld (ties %ld), mismatches %ld\n", checked, ties, bad);
    return bad ? 1 : 0;
}
