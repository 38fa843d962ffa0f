// Activation quantizer: rows of f32 activations to 8-bit blocks of 32 or 256
// (reference Q8.QuantizeBlocks, internal/kernels/q8.go:50-97, with
// amaxQ8Go/quantQ8Go/sumsQ8Go at q8.go:237-273).
//
// Per block: amax = max|x|; the row is refused (ok = 0) if any |x| is NaN or
// above 2^60; q = RoundToEven(127*x/amax) of the exact quotient (0 when
// amax == 0; quant_rne.hpp); d = f32(amax)/127 (correctly rounded f32
// division), stored for each run of 32; xs = sum of each run of 32;
// ys16 = sum of each run of 16 (used by the Q6_K kernels for the bias of
// 32); dbs = d*f32(xs).
//
// One workgroup per row, up to 16 waves; each wave takes one chunk of 256
// elements at a time (one block of 256, or eight blocks of 32), four
// elements per lane, float4 loads.
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// CPW chunks of 256 per wave, their loads all issued before any compute
// (one memory round trip per row instead of one per chunk).
template <int BLOCK, int CPW>
__global__ __launch_bounds__(1024) void quantize_act_kernel(const float* __restrict__ x, int64_t K,
                                                            ActPtrs a) {
    const int row = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    const float* xr = x + (int64_t)row * K;
    const int64_t R32 = K / 32, nch = (K + 255) / 256;
    bool bad = false;
    for (int64_t c0 = wave; c0 < nch; c0 += (int64_t)nwaves * CPW) {
    float4 vv[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        // clamped: a chunk past the end reloads the last one (not used)
        const int64_t c = min(c0 + nwaves * i, nch - 1);
        const int64_t e0 = min(c * 256 + 4 * lane, K - 4);
        vv[i] = *(const float4*)(xr + e0);
    }
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int64_t c = c0 + nwaves * i;
        if (c >= nch) break;  // uniform within the wave
        const int64_t e0 = c * 256 + 4 * lane;
        // blocks of 32: K is a multiple of 32, so each group of eight lanes
        // is wholly inside or outside the row (the DPP steps stay in-group)
        if (BLOCK == 32 && e0 >= K) continue;
        const float4 v = vv[i];
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
            m = fmaxf(m, __shfl_xor(m, 16));
            m = fmaxf(m, __shfl_xor(m, 32));
            amax = m;
            bbad = __any(lbad);
        } else {
            amax = group8_max(m);  // eight lanes hold one block of 32
            bbad = lbad;
        }
        bad |= bbad;
        const float xv[4] = {v.x, v.y, v.z, v.w};
        int qv[4];
        const bool quant = !bbad && amax > 0.f;
        const float inv = quant ? 1.0f / amax : 0.f;
        for (int k = 0; k < 4; k++) qv[k] = quant ? quant_rne(xv[k], amax, inv) : 0;
        uint32_t packed = (uint32_t)(qv[0] & 0xFF) | ((uint32_t)(qv[1] & 0xFF) << 8) |
                          ((uint32_t)(qv[2] & 0xFF) << 16) | ((uint32_t)(qv[3] & 0xFF) << 24);
        *(uint32_t*)(a.q + (int64_t)row * K + e0) = packed;
        int s4 = qv[0] + qv[1] + qv[2] + qv[3];
        // run of 16 = 4 lanes, run of 32 = 8 lanes
        int s16 = s4 + __builtin_amdgcn_mov_dpp(s4, DPP_QUAD_1032, 0xF, 0xF, false);
        s16 += __builtin_amdgcn_mov_dpp(s16, DPP_QUAD_2301, 0xF, 0xF, false);
        int s32 = s16 + __builtin_amdgcn_mov_dpp(s16, DPP_HALF_MIRROR, 0xF, 0xF, false);
        const float d = amax / 127.0f;
        const int64_t run = e0 / 32;
        if ((lane & 3) == 0) a.ys16[(int64_t)row * (K / 16) + e0 / 16] = (int16_t)s16;
        if ((lane & 7) == 0) {
            a.xs[row * R32 + run] = (int16_t)s32;
            a.d32[row * R32 + run] = d;
            a.dbs[row * R32 + run] = d * (float)(int16_t)s32;
        }
    }
    }
    int any_bad = __syncthreads_or(bad ? 1 : 0);
    if (threadIdx.x == 0) a.ok[row] = any_bad ? 0 : 1;
}

hipError_t launch_quantize_act(const float* x, int64_t rows, int64_t K, int block, const ActPtrs& a,
                               hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t chunks = (K + 255) / 256;
    const int waves = (int)(chunks < 16 ? chunks : 16);
    const int64_t cpw = (chunks + waves - 1) / waves;  // rounds of 8 beyond K = 32768
    dim3 grid((unsigned)rows), blk(64 * waves);
#define QA_LAUNCH(B, C) hipLaunchKernelGGL((quantize_act_kernel<B, C>), grid, blk, 0, stream, x, K, a)
    if (block == 256) {
        if (cpw == 1) QA_LAUNCH(256, 1);
        else if (cpw == 2) QA_LAUNCH(256, 2);
        else if (cpw <= 4) QA_LAUNCH(256, 4);
        else QA_LAUNCH(256, 8);
    } else {
        if (cpw == 1) QA_LAUNCH(32, 1);
        else if (cpw == 2) QA_LAUNCH(32, 2);
        else if (cpw <= 4) QA_LAUNCH(32, 4);
        else QA_LAUNCH(32, 8);
    }
#undef QA_LAUNCH
    return hipGetLastError();
}

}  // namespace mimg
