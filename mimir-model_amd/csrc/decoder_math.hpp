// Device math shared by the decoder ops and the activation quantizer: the
// reference's Cephes expf and silu product (internal/kernels/attn_amd64.s),
// and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimg {

// The key cache is [Hkv][C][D]. The value cache is blocked by eight keys:
// value (kv head hk, key j, dim d) at ((hk*ceil(C/8) + j/8)*D + d)*8 + j%8,
// so that one dim's eight consecutive keys are 16 contiguous bytes (f16) for
// the weighted sum, which runs one chain per dim in key order.
__host__ __device__ __forceinline__ int64_t vcache_at(int hk, int64_t j, int d, int D, int64_t C) {
    return (((int64_t)hk * ((C + 7) >> 3) + (j >> 3)) * D + d) * 8 + (j & 7);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Cephes' expf as the reference's expSumF32AVX2 evaluates it
// (attn_amd64.s:81-240): t clamped to lo, f = rint(t*log2e), r = t - f*ln2
// with ln2 in two parts (fma), exp(r) = 1 + r + r^2 P(r), times 2^f put in
// the exponent; t < lo (and NaN) gives 0.
__device__ __forceinline__ float cephes_exp(float t) {
    const float lo = __uint_as_float(0xc2aeac4fu), log2e = __uint_as_float(0x3fb8aa3bu);
    const float c1 = __uint_as_float(0x3f318000u), c2 = __uint_as_float(0xb95e8083u);
    const bool keep = t >= lo;
    const float tt = t > lo ? t : lo;
    const float f = __builtin_rintf(tt * log2e);
    float r = __builtin_fmaf(-f, c1, tt);
    r = __builtin_fmaf(-f, c2, r);
    const float r2 = r * r;
    float p = __uint_as_float(0x39506967u);
    p = __builtin_fmaf(p, r, __uint_as_float(0x3ab743ceu));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3c088908u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3d2aa9c1u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3e2aaaaau));
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r2, r);
    p = p + 1.0f;
    const float e = p * __uint_as_float((uint32_t)((int32_t)f + 127) << 23);
    return keep ? e : 0.0f;
}

// silu(x) * b as the reference's siluMulF32AVX2 (attn_amd64.s:459-535):
// h = exp(-|x|/2) by the Cephes steps, silu = x/(1+h*h) for x >= 0 and
// ((x*h)*h)/(1+h*h) below, then times b.
__device__ __forceinline__ float silu_mul_vec(float x, float b) {
    const float hh = cephes_exp(-__builtin_fabsf(x) * 0.5f);
    const float e1 = hh * hh + 1.0f;
    const float y = (x * hh) * hh;
    return ((x >= 0.f ? x : y) / e1) * b;
}

// swiglu.v1 element i of n, as the reference computes it with pieces of
// `chunk` elements (parallel(), interp/pool.go:33-51): the first len&~7 of
// a piece through the vector formula, the rest through float64
// (SiluMulF32, internal/kernels/attn.go:63-76).
__device__ __forceinline__ float swiglu_in_piece(float g, float u, int64_t i, int64_t lo, int64_t n, int64_t chunk) {
    const int64_t len = lo + chunk < n ? chunk : n - lo;
    const int64_t nv = len >= 8 ? (len & ~(int64_t)7) : 0;
    if (i - lo < nv) return silu_mul_vec(g, u);
    const double a = (double)g;
    return (float)(a / (1.0 + exp(-a)) * (double)u);
}
__device__ __forceinline__ int64_t piece_start(int64_t i, int64_t chunk) {
    // n < 2^32 in practice: a 32-bit division is far cheaper than a 64-bit one
    if (((uint64_t)i | (uint64_t)chunk) < 0x100000000ull) return (int64_t)((uint32_t)i / (uint32_t)chunk) * chunk;
    return i / chunk * chunk;
}
__device__ __forceinline__ float swiglu_at(float g, float u, int64_t i, int64_t n, int64_t chunk) {
    return swiglu_in_piece(g, u, i, piece_start(i, chunk), n, chunk);
}
// Four consecutive elements i..i+3: one division for the four.
__device__ __forceinline__ float4 swiglu4(float4 g, float4 u, int64_t i, int64_t n, int64_t chunk) {
    int64_t lo = piece_start(i, chunk);
    float4 o;
    o.x = swiglu_in_piece(g.x, u.x, i, lo, n, chunk);
    while (i + 1 - lo >= chunk) lo += chunk;
    o.y = swiglu_in_piece(g.y, u.y, i + 1, lo, n, chunk);
    while (i + 2 - lo >= chunk) lo += chunk;
    o.z = swiglu_in_piece(g.z, u.z, i + 2, lo, n, chunk);
    while (i + 3 - lo >= chunk) lo += chunk;
    o.w = swiglu_in_piece(g.w, u.w, i + 3, lo, n, chunk);
    return o;
}

}  // namespace mimg
