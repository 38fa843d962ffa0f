// Device helpers shared by the gfx950 kernels: block layouts, f16 decode,
// aligned loads of 2-byte-aligned blocks, and wavefront reductions.
//
// All kernels are compiled with -ffp-contract=off: every float multiply and
// add rounds separately unless __builtin_fmaf is written, so the float
// operation order of each kernel is the one its comment states.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimg {

// mim dtype ids (reference dtype.go:22-46).
enum : uint32_t { DT_F32 = 1, DT_Q8_0 = 64, DT_Q4_K = 66, DT_Q6_K = 67 };

// Block geometry (reference dtype.go:63-68, spec/dtypes.md).
constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;  // f16 d, f16 dmin, 12 scale bytes, 128 nibble bytes
constexpr int Q6K_BYTES = 210;  // 128 ql, 64 qh, 16 int8 scales, f16 d
constexpr int Q80_BYTES = 34;   // f16 d, 32 int8

// Device weight buffers are allocated this many bytes past their data so
// that the 20-byte window loads below never leave the allocation.
constexpr int WEIGHT_PAD = 256;

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// f16 bits to float32, exact (the hardware conversion keeps subnormals with
// the kernel's denormal mode "preserve", checked exhaustively by the tests).
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ bool f16_finite(uint32_t bits) { return (bits & 0x7C00u) != 0x7C00u; }

// 16 bytes starting at a 2-byte-aligned address: five aligned dwords, then
// byte realignment. Reads up to 4 bytes past p+16 (inside WEIGHT_PAD).
__device__ __forceinline__ u32x4 load16_a2(const uint8_t* p) {
    const uint32_t* b = (const uint32_t*)__builtin_align_down(p, 4);
    uint32_t s = (uint32_t)((uintptr_t)p & 3);
    u32x4a4 v = *(const u32x4a4*)b;
    uint32_t v4 = b[4];
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, s);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, s);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, s);
    r.w = __builtin_amdgcn_alignbyte(v4, v.w, s);
    return r;
}

// 4 bytes starting at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t load4_a2(const uint8_t* p) {
    const uint32_t* b = (const uint32_t*)__builtin_align_down(p, 4);
    uint32_t s = (uint32_t)((uintptr_t)p & 3);
    return __builtin_amdgcn_alignbyte(b[1], b[0], s);
}

__device__ __forceinline__ uint16_t load_u16(const uint8_t* p) { return *(const uint16_t*)p; }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// DPP controls (gfx9): quad permutes and the half-row mirror.
constexpr int DPP_QUAD_1032 = 0xB1;  // lanes [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;  // lanes [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <-> 15-i within a row of 16

__device__ __forceinline__ int dpp_i(int v, int ctrl) {
    switch (ctrl) {
    case DPP_QUAD_1032: return __builtin_amdgcn_mov_dpp(v, DPP_QUAD_1032, 0xF, 0xF, false);
    case DPP_QUAD_2301: return __builtin_amdgcn_mov_dpp(v, DPP_QUAD_2301, 0xF, 0xF, false);
    default: return __builtin_amdgcn_mov_dpp(v, DPP_HALF_MIRROR, 0xF, 0xF, false);
    }
}

// Sum of an int32 over each aligned group of 8 lanes, left in all 8 lanes.
// Integer addition is associative, so the result is exact in any order.
// (Every lane of these permutes has a source, so bound_ctrl changes nothing;
// with it set the compiler folds each move into the add, v_add_u32_dpp.)
__device__ __forceinline__ int group8_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, DPP_QUAD_1032, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_QUAD_2301, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_HALF_MIRROR, 0xF, 0xF, true);
    return v;
}

__device__ __forceinline__ float group8_max(float v) {
    int vi = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(vi, DPP_QUAD_1032, 0xF, 0xF, false)));
    vi = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(vi, DPP_QUAD_2301, 0xF, 0xF, false)));
    vi = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(vi, DPP_HALF_MIRROR, 0xF, 0xF, false)));
    return v;
}

// Q4_K: the eight 6-bit scales and the eight 6-bit mins of a block as bytes
// (reference getScaleMinK4, quant.go:272-281): from the scale dwords
// S0 = bytes 4..7, S1 = 8..11, S2 = 12..15 of the block.
struct Q4KScales {
    uint64_t sc;  // byte j = scale of sub-block j
    uint64_t m;   // byte j = min of sub-block j
};
__device__ __forceinline__ Q4KScales q4k_scales(uint32_t S0, uint32_t S1, uint32_t S2) {
    uint32_t sc_lo = S0 & 0x3F3F3F3Fu;
    uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    uint32_t m_lo = S1 & 0x3F3F3F3Fu;
    uint32_t m_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    Q4KScales r;
    r.sc = (uint64_t)sc_lo | ((uint64_t)sc_hi << 32);
    r.m = (uint64_t)m_lo | ((uint64_t)m_hi << 32);
    return r;
}

__device__ __forceinline__ uint32_t byte_of(uint64_t v, int j) { return (uint32_t)(v >> (8 * j)) & 0xFFu; }

// Packed 16-bit lanes (int8 MFMA operand building).
typedef short s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t as_u32(s16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) { return __builtin_bit_cast(s16x2, v); }

// A barrier for LDS only: it waits for this wave's LDS operations, not for
// its outstanding global loads and stores.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Whether p holds on any thread of the workgroup's nw waves: one LDS flag
// per wave (slot[nw], written once per launch) and one LDS-only barrier.
// (HIP's __syncthreads_or takes three barriers and first waits for every
// load and store the wave has in flight.)
__device__ __forceinline__ bool wg_any(bool p, int* slot, int nw) {
    const bool any = __any(p);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = any ? 1 : 0;
    lds_barrier();
    int r = 0;
    for (int i = 0; i < nw; i++) r |= slot[i];
    return r != 0;
}

}  // namespace mimg

#include "quant_rne.hpp"

namespace mimg {

}  // namespace mimg
