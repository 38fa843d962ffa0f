// The activation quantizer's rounding, shared by the GPU kernels and a CPU
// check (tests/test_quant_rne.py builds this header with g++): plain C++,
// host and device.
#pragma once

#if defined(__HIPCC__)
#define MIMG_HD __host__ __device__
#else
#define MIMG_HD
#endif

namespace mimg {

// RoundToEven(127*x/amax) of the exact quotient q* (the reference computes
// it in float64, whose rounding cannot change the result: q8.go:78-84), for
// 0 < amax, |x| <= amax <= 2^60, inv = 1/amax in f32.
// Fast path in float32 (amax >= 2^-120, so inv is finite): r = f32(127x) *
// inv is within 2^-15 of q* (three roundings of relative size 2^-24,
// |q*| <= 127; a subnormal 127x adds at most 2^-150 * inv <= 2^-30), so when
// r is more than 2^-12 away from a half-integer, rint(r) is the rounding of
// q*. Otherwise (and for tiny amax, from a float64 quotient) q* is compared
// exactly with the nearby half-integer h: the sign of fma(h, amax, -127x) in
// float64 (a correctly rounded difference has the exact one's sign and is
// zero only when it is) is that of h - q*; a zero is a tie, which goes to
// the even neighbour.
MIMG_HD inline int quant_rne(float x, float amax, float inv) {
    const double t = 127.0 * (double)x;  // exact
    double n, dd;
    if (amax >= 0x1p-120f) {
        const float rf = (127.0f * x) * inv;
        const float nf = __builtin_rintf(rf);
        const float df = rf - nf;  // exact (Sterbenz)
        if (__builtin_fabsf(df) <= 0.5f - 0x1p-12f) return (int)nf;
        n = nf;
        dd = df;
    } else {
        const double r = t / (double)amax;
        n = __builtin_rint(r);
        dd = r - n;
        if (__builtin_fabs(dd) <= 0.49) return (int)n;
    }
    const double h = n + (dd > 0.0 ? 0.5 : -0.5);
    const double e = __builtin_fma(h, (double)amax, -t);
    const double lo = h - 0.5;  // an integer in [-128, 128]
    double q;
    if (e > 0.0) q = lo;
    else if (e < 0.0) q = lo + 1.0;
    else q = ((int)lo & 1) == 0 ? lo : lo + 1.0;  // (even lo; f64 fmod is a slow software loop on the GPU)
    return (int)q;
}

// The fast path of quant_rne alone, branch-free: q = rint(f32(127x)*inv),
// and whether that is the rounding of q* (false: call quant_rne). Same
// expressions as quant_rne's fast path, so the two agree wherever this one
// answers.
MIMG_HD inline bool quant_rne_fast(float x, float amax, float inv, int& q) {
    const float rf = (127.0f * x) * inv;
    const float nf = __builtin_rintf(rf);
    const float df = rf - nf;  // exact (Sterbenz)
    const bool ok = amax >= 0x1p-120f && __builtin_fabsf(df) <= 0.5f - 0x1p-12f;
    q = ok ? (int)nf : 0;  // |nf| <= 127 when ok
    return ok;
}

}  // namespace mimg
