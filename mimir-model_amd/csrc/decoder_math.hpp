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

// The value of lane i ^ M (M a power of two below 64): DPP within a row of
// 16 lanes for M <= 8 (quad permutes for 1 and 2; row shifts of four into
// each half-row, by bank mask, for 4; a rotation by eight for 8), a
// swizzle within 32 lanes for 16, a permute for 32. The wave reductions
// below add (or take the max of) the same partners in the same order as a
// loop of __shfl_xor(v, M) for M = 32, 16, ..., 1, so their results are
// the same bits.
template <int M>
__device__ __forceinline__ int lane_xor(int x) {
    if constexpr (M == 1) return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    else if constexpr (M == 2) return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else if constexpr (M == 4) {
        const int t = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xA, false);  // row_shr:4 into lanes 4-7, 12-15
        return __builtin_amdgcn_update_dpp(t, x, 0x104, 0xF, 0x5, false);         // row_shl:4 into lanes 0-3, 8-11
    } else if constexpr (M == 8) return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
    else if constexpr (M == 16) return __builtin_amdgcn_ds_swizzle(x, 0x401F);  // bit-mask mode: lane ^ 16
    else return __shfl_xor(x, 32);
}
template <int M>
__device__ __forceinline__ float lane_xor_f32(float v) {
    return __int_as_float(lane_xor<M>(__float_as_int(v)));
}
template <int M>
__device__ __forceinline__ double lane_xor_f64(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = lane_xor<M>((int)(b & 0xFFFFFFFFll)), hi = lane_xor<M>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += lane_xor_f64<32>(v);
    v += lane_xor_f64<16>(v);
    v += lane_xor_f64<8>(v);
    v += lane_xor_f64<4>(v);
    v += lane_xor_f64<2>(v);
    v += lane_xor_f64<1>(v);
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += lane_xor_f32<32>(v);
    v += lane_xor_f32<16>(v);
    v += lane_xor_f32<8>(v);
    v += lane_xor_f32<4>(v);
    v += lane_xor_f32<2>(v);
    v += lane_xor_f32<1>(v);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, lane_xor_f32<32>(v));
    v = fmaxf(v, lane_xor_f32<16>(v));
    v = fmaxf(v, lane_xor_f32<8>(v));
    v = fmaxf(v, lane_xor_f32<4>(v));
    v = fmaxf(v, lane_xor_f32<2>(v));
    v = fmaxf(v, lane_xor_f32<1>(v));
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
