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
// Work split: a wave takes one chunk of 256 elements at a time (one block of
// 256, or eight blocks of 32), four elements per lane, float4 loads. rms_norm
// (which needs the whole row's sum of squares first) runs one workgroup per
// row of up to 16 waves; the plain quantizer and swiglu run eight chunks per
// workgroup, many workgroups per row.
#include "decoder_math.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"
#include "qa_chunk.hpp"

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
    const int64_t nch = (K + 255) / 256;
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
        bad |= qa_chunk<BLOCK>(vv[i], row, c * 256 + 4 * lane, K, a, lane);
    }
    }
    __shared__ int wflag[16];
    const bool any_bad = wg_any(bad, wflag, (int)(blockDim.x >> 6));
    if (threadIdx.x == 0) a.ok[row] = any_bad ? 0 : 1;
}

// Many workgroups per row (QA_PLAIN, QA_SWIGLU): workgroup 1+gi of a row
// quantizes chunks 8gi..8gi+7, one per wave. The row's refusal flag depends
// on the whole row, so workgroup 0 of each row only scans it, all its loads
// in one round for K <= 16384: QA_PLAIN tests every x; QA_SWIGLU screens g
// and u, and computes y exactly (swiglu_at, as written) only where the
// screen does not pass. Screen: g and u finite with |g|, |u| <= 2^29. Then
// |silu(g)| <= |g| in both of the reference's formulas (the vector one
// divides (g*h)*h or g, h = exp(-|g|/2) <= 1, by h*h + 1 >= 1; the scalar one
// divides by 1 + exp(-g) >= 1), so |y| <= 2^58 < 2^60 and y is not NaN: such
// elements never refuse a row.
constexpr int QA_MW_WAVES = 8;  // chunks of 256 per workgroup, one per wave

template <int BLOCK, int MODE>
__global__ __launch_bounds__(64 * QA_MW_WAVES) void quantize_act_mw_kernel(const float* __restrict__ x, int64_t K,
                                                                           ActPtrs a, QaSource src) {
    static_assert(MODE == QA_PLAIN || MODE == QA_SWIGLU, "rms_norm needs the whole row first");
    const int row = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t nch = (K + 255) / 256;
    const float* xr = x + (int64_t)row * K;
    const float* ur = MODE == QA_SWIGLU ? src.aux + (int64_t)row * K : nullptr;
    if (blockIdx.x > 0) {
        const int64_t c = (int64_t)(blockIdx.x - 1) * QA_MW_WAVES + wave;
        if (c >= nch) return;  // uniform within the wave
        const int64_t e0 = c * 256 + 4 * lane, el = min(e0, K - 4);
        float4 v = *(const float4*)(xr + el);
        if constexpr (MODE == QA_SWIGLU) {
            const float4 uu = *(const float4*)(ur + el);
            const int64_t gi = (int64_t)row * K + el;
            v = swiglu4(v, uu, gi, src.total, src.chunk);
            if (e0 < K) *(float4*)(src.y + gi) = v;
        }
        qa_chunk<BLOCK>(v, row, e0, K, a, lane);
        return;
    }
    // SCAN float4 loads of x (and of u) per thread in flight, clamped and
    // checked where inside the row, in straight-line code (registers).
    constexpr int SCAN = 8, STEP = 4 * 64 * QA_MW_WAVES;
    bool bad = false;
    for (int64_t e0 = 4 * (int64_t)threadIdx.x; e0 < K; e0 += (int64_t)STEP * SCAN) {
        float4 v[SCAN], w[MODE == QA_SWIGLU ? SCAN : 1];
#pragma unroll
        for (int j = 0; j < SCAN; j++) {
            const int64_t e = min(e0 + (int64_t)STEP * j, K - 4);
            v[j] = *(const float4*)(xr + e);
            if constexpr (MODE == QA_SWIGLU) w[j] = *(const float4*)(ur + e);
        }
#pragma unroll
        for (int j = 0; j < SCAN; j++) {
            const int64_t e = e0 + (int64_t)STEP * j;
            if (e >= K) continue;
            const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            if constexpr (MODE == QA_PLAIN) {
#pragma unroll
                for (int k = 0; k < 4; k++) bad |= !(fabsf(xv[k]) <= 0x1p60f);
            } else {
                const float uv[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (fabsf(xv[k]) <= 0x1p29f && fabsf(uv[k]) <= 0x1p29f) continue;
                    const float y = swiglu_at(xv[k], uv[k], (int64_t)row * K + e + k, src.total, src.chunk);
                    bad |= !(fabsf(y) <= 0x1p60f);
                }
            }
        }
    }
    const int any_bad = __syncthreads_or(bad ? 1 : 0);
    if (threadIdx.x == 0) a.ok[row] = any_bad ? 0 : 1;
}

template <int MODE>
static hipError_t launch_qa(const float* x, int64_t rows, int64_t K, int block, const ActPtrs& a, const QaSource& src,
                            hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t chunks = (K + 255) / 256;
    // Rows of at most 16 chunks (K <= 4096), and any row of a call with 64
    // rows or more, take one workgroup of up to 16 waves: no scanning
    // workgroup reads the row a second time, and the refusal flag is one LDS
    // vote (measured on MI355X: the cfg1 step 51.2 -> 50.8 us, 8B decode
    // batch 8 +0.9 %; the 8B prompt of 512 rows +3 % with swiglu + quantize
    // at K = 14336 so). Few long rows keep many workgroups a row (one
    // workgroup a row at K = 14336 made the 8B decode step 2.7 % slower).
    constexpr int64_t one_wg = 16;
    const bool fits_one = MODE == QA_PLAIN || chunks <= 16 * 8;  // swiglu: one round of loads
    if (MODE != QA_NORM && rows <= 65535 && chunks > one_wg && (rows < 64 || !fits_one)) {
        dim3 grid((unsigned)(1 + (chunks + QA_MW_WAVES - 1) / QA_MW_WAVES), (unsigned)rows), blk(64 * QA_MW_WAVES);
        if (block == 256)
            hipLaunchKernelGGL((quantize_act_mw_kernel<256, MODE == QA_NORM ? QA_PLAIN : MODE>), grid, blk, 0, stream,
                               x, K, a, src);
        else
            hipLaunchKernelGGL((quantize_act_mw_kernel<32, MODE == QA_NORM ? QA_PLAIN : MODE>), grid, blk, 0, stream,
                               x, K, a, src);
        return hipGetLastError();
    }
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

// Rows of different K, each with its own ActPtrs, in one launch (the inputs
// of a set of independent products, mimg_linear_a8_set_dev), blocks of 256.
// Row i owns workgroups wg0 .. wg0 + ceil(chunks/8): the first scans the row
// for the refusal flag, the others quantize eight chunks each, exactly as
// quantize_act_mw_kernel<256, QA_PLAIN> does for a row on its own.
__global__ __launch_bounds__(64 * QA_MW_WAVES) void quantize_act_set_kernel(QaSetArgs args) {
    const QaSetArgs* S = (const QaSetArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    const int bid = (int)blockIdx.x;
    int ri = 0;
    for (int i = 1; i < S->nrows; i++) ri = bid >= S->row[i].wg0 ? i : ri;
    const QaSetRow* r = &S->row[ri];
    const int64_t K = r->K, nch = (K + 255) / 256;
    const float* xr = r->x;
    const ActPtrs a = r->a;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, gi = bid - r->wg0;
    if (gi > 0) {
        const int64_t c = (int64_t)(gi - 1) * QA_MW_WAVES + wave;
        if (c >= nch) return;  // uniform within the wave
        const int64_t e0 = c * 256 + 4 * lane, el = min(e0, K - 4);
        const float4 v = *(const float4*)(xr + el);
        qa_chunk<256>(v, 0, e0, K, a, lane);
        return;
    }
    constexpr int SCAN = 8, STEP = 4 * 64 * QA_MW_WAVES;
    bool bad = false;
    for (int64_t e0 = 4 * (int64_t)threadIdx.x; e0 < K; e0 += (int64_t)STEP * SCAN) {
        float4 v[SCAN];
#pragma unroll
        for (int j = 0; j < SCAN; j++) v[j] = *(const float4*)(xr + min(e0 + (int64_t)STEP * j, K - 4));
#pragma unroll
        for (int j = 0; j < SCAN; j++) {
            if (e0 + (int64_t)STEP * j >= K) continue;
            const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int k = 0; k < 4; k++) bad |= !(fabsf(xv[k]) <= 0x1p60f);
        }
    }
    const int any_bad = __syncthreads_or(bad ? 1 : 0);
    if (threadIdx.x == 0) a.ok[0] = any_bad ? 0 : 1;
}

hipError_t launch_quantize_act_set(const QaSetArgs& a, int wgs, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_act_set_kernel, dim3((unsigned)wgs), dim3(64 * QA_MW_WAVES), 0, stream, a);
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
