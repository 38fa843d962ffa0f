// Float32-activation dot products (dequant_matmul.v1 and the fallback of the
// 8-bit path), computed by a group of eight lanes in the float order of the
// reference's AVX2 kernels: lane l of the group is SIMD lane l, holding the
// four accumulators Y0..Y3 of that lane, and the final sum is the
// reference's HSUM (internal/kernels/kernels_amd64.s:28-37).
//
//   fused (a row used at most DecodeOnce = 8 times, kernels.go:83-100):
//     Q4_K dotQ4KAVX2 (kernels_amd64.s:112-170), Q6_K dotQ6KAVX2 (:172-282),
//     Q8_0 dotQ8_0AVX2 (:284-308); each weight decoded with the float ops of
//     mim.Dequantize, then one fused multiply-add into its lane.
//   not fused (Load decodes the row, then DotF32, kernels.go:37-49 with
//     dotF32AVX2, kernels_amd64.s:45-85): element 32s+8r+l goes to Y_r of
//     lane l, for K a multiple of 32.
#pragma once

#include "mimg_device.hpp"

namespace mimg {

// Exact decode of one weight (reference quant.go:197-206, 283-344): the
// float32 operations of mim.Dequantize in its order, each rounded.
__device__ __forceinline__ float q4k_weight(const uint8_t* blk, int e) {
    float d = f16_to_f32(load_u16(blk)), dmin = f16_to_f32(load_u16(blk + 2));
    const uint8_t* s = blk + 4;
    int sb = e >> 5;
    uint32_t sc, m;
    if (sb < 4) {
        sc = s[sb] & 63;
        m = s[sb + 4] & 63;
    } else {
        sc = (s[sb + 4] & 0xF) | ((s[sb - 4] >> 6) << 4);
        m = (s[sb + 4] >> 4) | ((s[sb] >> 6) << 4);
    }
    int c = e >> 6, i = e & 63;
    uint32_t byte = blk[16 + 32 * c + (i & 31)];
    uint32_t q = i < 32 ? (byte & 0xF) : (byte >> 4);
    float ds = d * (float)sc;
    float ms = dmin * (float)m;
    return ds * (float)q - ms;
}

__device__ __forceinline__ float q6k_weight(const uint8_t* blk, int e) {
    float d = f16_to_f32(load_u16(blk + 208));
    int h = e >> 7, r = e & 127, p = r >> 5, l = r & 31;
    const uint8_t* ql = blk + 64 * h;
    const uint8_t* qh = blk + 128 + 32 * h;
    int v;
    switch (p) {
    case 0: v = (ql[l] & 0xF) | ((qh[l] & 3) << 4); break;
    case 1: v = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4); break;
    case 2: v = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4); break;
    default: v = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4); break;
    }
    float s = d * (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * p];
    return s * (float)(v - 32);
}

__device__ __forceinline__ float q8_0_weight(const uint8_t* blk, int e) {
    return f16_to_f32(load_u16(blk)) * (float)(int8_t)blk[2 + e];
}

template <uint32_t DT>
__device__ __forceinline__ float decode_weight(const uint8_t* row, int64_t e) {
    if (DT == DT_Q4_K) return q4k_weight(row + (e >> 8) * Q4K_BYTES, (int)(e & 255));
    if (DT == DT_Q6_K) return q6k_weight(row + (e >> 8) * Q6K_BYTES, (int)(e & 255));
    return q8_0_weight(row + (e >> 5) * Q80_BYTES, (int)(e & 31));
}

// The reference HSUM over the eight lanes of the calling group (all eight
// lanes must be active); the result is returned in every lane of the group.
__device__ __forceinline__ float hsum_group8(float y0, float y1, float y2, float y3) {
    const int lane = threadIdx.x & 63, base = lane & ~7, l = lane & 7;
    float t = (y0 + y1) + (y2 + y3);
    float c = t + __shfl(t, base + ((l + 4) & 7));   // c_l = T_l + T_{l+4}, l < 4
    float e = c + __shfl(c, base + ((l + 1) & 7));   // e_0 = c0+c1, e_2 = c2+c3
    float r = e + __shfl(e, base + ((l + 2) & 7));   // r_0 = e_0 + e_2
    return __shfl(r, base);
}

// The float32 dot product of one weight row (K elements of dtype DT) with x,
// in the reference's order; called by all eight lanes of a group. It serves
// refused rows only, so it is written for few live registers (loops kept
// rolled, each chunk's scales decoded once) rather than speed: it is inlined
// into the 8-bit kernels and must not raise their register count.
// A read of x: plain, or (COH) an agent-scope load that sees stores made
// by other workgroups of the same launch (a row produced inside a kernel).
template <bool COH>
__device__ __forceinline__ float ldx(const float* p) {
    if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}

template <uint32_t DT, bool COH = false>
__device__ float f32dot_g8(const uint8_t* row, const float* x, int64_t K, bool fused) {
    const int l = threadIdx.x & 7;
    float Y[4] = {0.f, 0.f, 0.f, 0.f};
    if (!fused) {
#pragma unroll 1
        for (int64_t s = 0; s < K / 32; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int64_t e = 32 * s + 8 * r + l;
                Y[r] = __builtin_fmaf(ldx<COH>(x + e), decode_weight<DT>(row, e), Y[r]);
            }
    } else if (DT == DT_Q4_K) {
#pragma unroll 1
        for (int64_t b = 0; b < K / 256; b++) {
            const uint8_t* blk = row + b * Q4K_BYTES;
            const float d = f16_to_f32(load_u16(blk)), dmin = f16_to_f32(load_u16(blk + 2));
#pragma unroll 1
            for (int c = 0; c < 4; c++) {
                // chunk c: sub-blocks 2c (low nibbles) and 2c+1 (high nibbles)
                const uint8_t* s = blk + 4;
                uint32_t sc0, m0, sc1, m1;
                if (c < 2) {
                    sc0 = s[2 * c] & 63, m0 = s[2 * c + 4] & 63;
                    sc1 = s[2 * c + 1] & 63, m1 = s[2 * c + 5] & 63;
                } else {
                    const int j0 = 2 * c, j1 = 2 * c + 1;
                    sc0 = (s[j0 + 4] & 0xF) | ((s[j0 - 4] >> 6) << 4), m0 = (s[j0 + 4] >> 4) | ((s[j0] >> 6) << 4);
                    sc1 = (s[j1 + 4] & 0xF) | ((s[j1 - 4] >> 6) << 4), m1 = (s[j1 + 4] >> 4) | ((s[j1] >> 6) << 4);
                }
                const float s0 = d * (float)sc0, o0 = dmin * (float)m0;
                const float s1 = d * (float)sc1, o1 = dmin * (float)m1;
                const uint8_t* q = blk + 16 + 32 * c;
                const float* xc = x + 256 * b + 64 * c;
#pragma unroll 1
                for (int st = 0; st < 4; st++) {
                    const int i = 8 * st + l, ra = (st & 1) ? 2 : 0;
                    const uint32_t byte = q[i];
                    const float wl = s0 * (float)(byte & 0xF) - o0;
                    const float wh = s1 * (float)(byte >> 4) - o1;
                    Y[ra] = __builtin_fmaf(wl, ldx<COH>(xc + i), Y[ra]);
                    Y[ra + 1] = __builtin_fmaf(wh, ldx<COH>(xc + 32 + i), Y[ra + 1]);
                }
            }
        }
    } else if (DT == DT_Q6_K) {
#pragma unroll 1
        for (int64_t b = 0; b < K / 256; b++)
#pragma unroll 1
            for (int h = 0; h < 2; h++)
#pragma unroll 1
                for (int st = 0; st < 4; st++)
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        int e = 128 * h + 32 * p + 8 * st + l;
                        float w = q6k_weight(row + b * Q6K_BYTES, e);
                        Y[p] = __builtin_fmaf(w, ldx<COH>(x + 256 * b + e), Y[p]);
                    }
    } else {
#pragma unroll 1
        for (int64_t b = 0; b < K / 32; b++) {
            const float d = f16_to_f32(load_u16(row + b * Q80_BYTES));
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float w = d * (float)(int8_t)row[b * Q80_BYTES + 2 + 8 * r + l];
                Y[r] = __builtin_fmaf(w, ldx<COH>(x + 32 * b + 8 * r + l), Y[r]);
            }
        }
    }
    return hsum_group8(Y[0], Y[1], Y[2], Y[3]);
}

}  // namespace mimg
