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
#include "decoder_math.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// CPW chunks of 256 per wave, their loads all issued before any compute
// (one memory round trip per row instead of one per chunk).
//
// MODE says what produces the row that is quantized (the op before the
// linear layer in the graph, importer/llama.go:317-547), so that it runs in
// the same launch, with the same results as on its own:
//   QA_PLAIN   the row x itself
//   QA_NORM    rms_norm.v1 (interp/fast.go:434-485): x += resid (written
//              back when resid is given), y = (x * inv) * scale with
//              inv = f32(1/sqrt(f64(f32(ss/K)) + f64(eps))), ss the f64 sum
//              of squares; y is written and quantized
//   QA_SWIGLU  swiglu.v1: y = silu(g) * u over the whole rows*K array with
//              the reference's pieces (swiglu_at); y is written and quantized
// The produced row must fit in one round of loads (K <= 16*CPW*256).
enum { QA_PLAIN = 0, QA_NORM = 1, QA_SWIGLU = 2 };

template <int BLOCK, int CPW, int MODE>
__global__ __launch_bounds__(1024) void quantize_act_kernel(const float* __restrict__ x, int64_t K,
                                                            ActPtrs a, QaSource src) {
    __shared__ double qa_part[16];
    const int row = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    const float* xr = x + (int64_t)row * K;
    const int64_t R32 = K / 32, nch = (K + 255) / 256;
    bool bad = false;
    for (int64_t c0 = wave; c0 < nch; c0 += (int64_t)nwaves * CPW) {
    float4 vv[CPW];
    float4 aux[MODE == QA_PLAIN ? 1 : CPW], scl[MODE == QA_NORM ? CPW : 1];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        // clamped: a chunk past the end reloads the last one (not used)
        const int64_t c = min(c0 + nwaves * i, nch - 1);
        const int64_t e0 = min(c * 256 + 4 * lane, K - 4);
        vv[i] = *(const float4*)(xr + e0);
        if constexpr (MODE == QA_NORM) {
            if (src.aux) aux[i] = *(const float4*)(src.aux + (int64_t)row * K + e0);
            if (src.scale) scl[i] = *(const float4*)(src.scale + e0);
        }
        if constexpr (MODE == QA_SWIGLU) aux[i] = *(const float4*)(src.aux + (int64_t)row * K + e0);
    }
    if constexpr (MODE != QA_PLAIN) {
        // one round: every wave is here once, so the group may synchronise
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const int64_t c = c0 + nwaves * i;
            const int64_t e0 = c * 256 + 4 * lane;
            const bool live = c < nch && e0 < K;
            if constexpr (MODE == QA_NORM) {
                if (src.aux) {
                    vv[i].x = vv[i].x + aux[i].x;
                    vv[i].y = vv[i].y + aux[i].y;
                    vv[i].z = vv[i].z + aux[i].z;
                    vv[i].w = vv[i].w + aux[i].w;
                    if (live) *(float4*)((float*)xr + e0) = vv[i];
                }
                if (live)
                    ss += (double)vv[i].x * (double)vv[i].x + (double)vv[i].y * (double)vv[i].y +
                          (double)vv[i].z * (double)vv[i].z + (double)vv[i].w * (double)vv[i].w;
            } else {
                const int64_t gi = (int64_t)row * K + (live ? e0 : 0);
                vv[i] = swiglu4(vv[i], aux[i], gi, src.total, src.chunk);
                if (live) *(float4*)(src.y + gi) = vv[i];
            }
        }
        if constexpr (MODE == QA_NORM) {
            ss = wave_sum_f64(ss);
            if (lane == 0) qa_part[wave] = ss;
            __syncthreads();
            double tot = 0.0;
            for (int w = 0; w < nwaves; w++) tot += qa_part[w];
            const float inv = (float)(1.0 / sqrt((double)(float)(tot / (double)K) + (double)src.eps));
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int64_t c = c0 + nwaves * i;
                const int64_t e0 = c * 256 + 4 * lane;
                float4 o = {vv[i].x * inv, vv[i].y * inv, vv[i].z * inv, vv[i].w * inv};
                if (src.scale) {
                    o.x = o.x * scl[i].x;
                    o.y = o.y * scl[i].y;
                    o.z = o.z * scl[i].z;
                    o.w = o.w * scl[i].w;
                }
                vv[i] = o;
                if (c < nch && e0 < K) *(float4*)(src.y + (int64_t)row * K + e0) = o;
            }
        }
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

template <int MODE>
static hipError_t launch_qa(const float* x, int64_t rows, int64_t K, int block, const ActPtrs& a, const QaSource& src,
                            hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t chunks = (K + 255) / 256;
    const int waves = (int)(chunks < 16 ? chunks : 16);
    const int64_t cpw = (chunks + waves - 1) / waves;  // rounds of 8 beyond K = 32768
    if (MODE != QA_PLAIN && cpw > 8) return hipErrorInvalidValue;
    dim3 grid((unsigned)rows), blk(64 * waves);
#define QA_LAUNCH(B, C) hipLaunchKernelGGL((quantize_act_kernel<B, C, MODE>), grid, blk, 0, stream, x, K, a, src)
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

hipError_t launch_quantize_act(const float* x, int64_t rows, int64_t K, int block, const ActPtrs& a,
                               hipStream_t stream) {
    return launch_qa<QA_PLAIN>(x, rows, K, block, a, QaSource{}, stream);
}

hipError_t launch_norm_quantize_act(float* x, const float* resid, const float* scale, float eps, float* y,
                                    int64_t rows, int64_t K, int block, const ActPtrs& a, hipStream_t stream) {
    QaSource src{};
    src.aux = resid;
    src.scale = scale;
    src.eps = eps;
    src.y = y;
    return launch_qa<QA_NORM>(x, rows, K, block, a, src, stream);
}

hipError_t launch_swiglu_quantize_act(const float* g, const float* u, float* y, int64_t chunk, int64_t rows,
                                      int64_t K, int block, const ActPtrs& a, hipStream_t stream) {
    QaSource src{};
    src.aux = u;
    src.y = y;
    src.chunk = chunk;
    src.total = rows * K;
    return launch_qa<QA_SWIGLU>(g, rows, K, block, a, src, stream);
}

}  // namespace mimg
