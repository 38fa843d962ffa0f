// One chunk of the activation quantizer (reference Q8.QuantizeBlocks,
// internal/kernels/q8.go:50-97), shared by the quantizer launches and the
// kernels that quantize their input row themselves. `a` may point into
// device memory or into the calling workgroup's LDS; a.dbs may be null
// (the per-32 products d*xs are then not written).
#pragma once

#include "decoder_math.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// Quantizes one chunk of 256 elements of row `row` (four per lane, lane's
// first element e0; all 64 lanes of the wave call it) and returns whether a
// lane's elements refuse the row (NaN or |x| > 2^60). The chunk's outputs
// depend on its own elements only.
template <int BLOCK>
__device__ __forceinline__ bool qa_chunk(const float4 v, int64_t row, int64_t e0, int64_t K, const ActPtrs& a,
                                         int lane) {
    const int64_t R32 = K / 32;
    // blocks of 32: K is a multiple of 32, so each group of eight lanes is
    // wholly inside or outside the row (the DPP steps stay in-group)
    if (BLOCK == 32 && e0 >= K) return false;
    float av[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
    bool lbad = false;
    float m = 0.f;
    for (int k = 0; k < 4; k++) {
        lbad |= !(av[k] <= 0x1p60f);
        m = fmaxf(m, av[k]);
    }
    float amax;
    bool bbad;
    if (BLOCK == 256) {
        // max over the wave; fmaxf of non-negative finite values is exact
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_QUAD_1032, 0xF, 0xF, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_QUAD_2301, 0xF, 0xF, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_HALF_MIRROR, 0xF, 0xF, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_ROW_MIRROR, 0xF, 0xF, false)));
        m = fmaxf(m, lane_xor_f32<16>(m));
        m = fmaxf(m, lane_xor_f32<32>(m));
        amax = m;
        bbad = __any(lbad);
    } else {
        amax = group8_max(m);  // eight lanes hold one block of 32
        bbad = lbad;
    }
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int qv[4];
    const bool quant = !bbad && amax > 0.f;
    const float inv = quant ? 1.0f / amax : 0.f;
    bool fast[4];
#pragma unroll
    for (int k = 0; k < 4; k++) fast[k] = quant_rne_fast(xv[k], amax, inv, qv[k]);
#pragma unroll
    for (int k = 0; k < 4; k++) qv[k] = !quant ? 0 : fast[k] ? qv[k] : quant_rne(xv[k], amax, inv);
    uint32_t packed = (uint32_t)(qv[0] & 0xFF) | ((uint32_t)(qv[1] & 0xFF) << 8) |
                      ((uint32_t)(qv[2] & 0xFF) << 16) | ((uint32_t)(qv[3] & 0xFF) << 24);
    *(uint32_t*)(a.q + row * K + e0) = packed;
    int s4 = qv[0] + qv[1] + qv[2] + qv[3];
    // run of 16 = 4 lanes, run of 32 = 8 lanes
    int s16 = s4 + __builtin_amdgcn_mov_dpp(s4, DPP_QUAD_1032, 0xF, 0xF, false);
    s16 += __builtin_amdgcn_mov_dpp(s16, DPP_QUAD_2301, 0xF, 0xF, false);
    int s32 = s16 + __builtin_amdgcn_mov_dpp(s16, DPP_HALF_MIRROR, 0xF, 0xF, false);
    const float d = amax / 127.0f;
    const int64_t run = e0 / 32;
    if ((lane & 3) == 0) a.ys16[row * (K / 16) + e0 / 16] = (int16_t)s16;
    if ((lane & 7) == 0) {
        a.xs[row * R32 + run] = (int16_t)s32;
        a.d32[row * R32 + run] = d;
        if (a.dbs) a.dbs[row * R32 + run] = d * (float)(int16_t)s32;
    }
    return bbad;
}

}  // namespace mimg
