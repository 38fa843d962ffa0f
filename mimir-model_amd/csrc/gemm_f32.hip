// Prefill product with float32 activations (dequant_matmul.v1, reference
// linearF32/linearCols, interp/fast.go:161-183) on the fp32 matrix cores:
// y[m][n] = sum_k x[m][k] * w[n][k] (+ bias[n]), w the decoded weights.
//
// Numerics. Each weight is decoded with the float32 operations of
// mim.Dequantize, bit for bit (f32path.hpp). The products and their sum
// run on v_mfma_f32_16x16x4_f32 in float32, K in steps of 4 per
// instruction, one accumulator per output over the whole of K; the bias is
// added to the finished sum, as the reference does. The summation order is
// not the reference's: the result is within the spec's bound for
// dequant_matmul.v1, |y - exact| <= (K+1) u sum_k |x_k w_k| with
// u = 2^-24 (spec/stdlib.md:230-246), which any float32 order of the K
// products meets (the tests check it against an exact sum). Products below
// the float32 normal range may be flushed by the matrix cores; the bound is
// not claimed for a sum made of such products only.
//
// Tiling: a 256-thread workgroup computes 128 weight rows x BM activation
// rows (BM = 128, or 64 when the 128-row tiles would leave CUs idle), K in
// stages of 32. Per stage every thread decodes 16 weights of one
// row and loads 16 activations of one row, both into LDS ([row][k], row
// stride 34 floats: the MFMA operand reads of a half-wave, 16 rows x 2 k,
// fall in 32 distinct banks); the four waves then run 4*BM/32 MFMAs per 4 k
// each on their 64 x BM/2 quarter. LDS is double-buffered: the global loads of
// stage s+1 are issued before the MFMAs of stage s and decoded into the
// other buffer after them, one barrier per stage.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

namespace {

constexpr int GF_BN = 128, GF_BK = 32, GF_S = GF_BK + 2;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One thread's share of a stage's weights: 16 consecutive k of row n,
// raw bytes as loaded (decoded after the MFMAs of the previous stage).
struct WRaw {
    u32x4 a, b;       // Q4_K: header, quant bytes; Q6_K: ql run, qh run; Q8_0: quant run
    uint32_t c, d;    // Q6_K: the fifth dwords of the ql and qh windows; Q8_0: the fifth dword
    uint32_t s;       // Q6_K: scale byte; Q8_0: d bits
    uint32_t e;       // Q6_K: d bits; the shift of 2-byte-aligned runs
};

// Stage k0 (a multiple of 32) of row `row`, elements k0 + 16h .. +16.
template <uint32_t DT>
__device__ __forceinline__ WRaw load_w(const uint8_t* row, int64_t k0, int h) {
    WRaw r;
    if constexpr (DT == DT_Q4_K) {
        const uint8_t* blk = row + (k0 >> 8) * Q4K_BYTES;
        const int j = (int)(k0 & 255) >> 5;  // sub-block
        r.a = *(const u32x4*)blk;
        r.b = *(const u32x4*)(blk + 16 + 32 * (j >> 1) + 16 * h);
    } else if constexpr (DT == DT_Q6_K) {
        const uint8_t* blk = row + (k0 >> 8) * Q6K_BYTES;
        const int j = (int)(k0 & 255) >> 5, hh = j >> 2, p = j & 3;
        const uint8_t* ql = blk + 64 * hh + ((p & 1) ? 32 : 0) + 16 * h;
        const uint8_t* qh = blk + 128 + 32 * hh + 16 * h;
        const uint32_t* qa = (const uint32_t*)__builtin_align_down(ql, 4);
        const uint32_t* qb = (const uint32_t*)__builtin_align_down(qh, 4);
        r.a = *(const u32x4a4*)qa;
        r.c = qa[4];
        r.b = *(const u32x4a4*)qb;
        r.d = qb[4];
        r.s = (uint32_t)blk[192 + 8 * hh + h + 2 * p];
        r.e = load_u16(blk + 208) | ((uint32_t)((uintptr_t)blk & 3) << 16);
    } else {
        const uint8_t* blk = row + (k0 >> 5) * Q80_BYTES;
        const uint32_t* qa = (const uint32_t*)__builtin_align_down(blk + 2 + 16 * h, 4);
        r.a = *(const u32x4a4*)qa;
        r.c = qa[4];
        r.s = load_u16(blk);
        r.e = (uint32_t)((uintptr_t)(blk + 2) & 3);
    }
    return r;
}

__device__ __forceinline__ u32x4 realign(const u32x4& v, uint32_t v4, uint32_t s) {
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, s);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, s);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, s);
    r.w = __builtin_amdgcn_alignbyte(v4, v.w, s);
    return r;
}

// The 16 weights of a thread's share, each with mim.Dequantize's float ops
// (the same expressions as q4k_weight / q6k_weight / q8_0_weight).
template <uint32_t DT>
__device__ __forceinline__ void decode_w(const WRaw& r, int64_t k0, float* out) {
    const int j = (int)(k0 & 255) >> 5;
    if constexpr (DT == DT_Q4_K) {
        const float d = f16_to_f32(r.a.x & 0xFFFFu), dmin = f16_to_f32(r.a.x >> 16);
        const Q4KScales s = q4k_scales(r.a.y, r.a.z, r.a.w);
        const float ds = d * (float)byte_of(s.sc, j), ms = dmin * (float)byte_of(s.m, j);
        const uint32_t q[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const int sh = (j & 1) * 4;
#pragma unroll
        for (int i = 0; i < 16; i++) out[i] = ds * (float)((q[i >> 2] >> (8 * (i & 3) + sh)) & 0xFu) - ms;
    } else if constexpr (DT == DT_Q6_K) {
        const uint32_t sh = r.e >> 16, p = (uint32_t)j & 3;
        const u32x4 ql = realign(r.a, r.c, sh), qh = realign(r.b, r.d, sh);
        const uint32_t lq[4] = {ql.x, ql.y, ql.z, ql.w}, hq[4] = {qh.x, qh.y, qh.z, qh.w};
        const float s = f16_to_f32(r.e & 0xFFFFu) * (float)(int8_t)r.s;
        const int lsh = (p >= 2) ? 4 : 0, hsh = 2 * (int)p;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int lo = (int)((lq[i >> 2] >> (8 * (i & 3) + lsh)) & 0xFu);
            const int hi = (int)((hq[i >> 2] >> (8 * (i & 3) + hsh)) & 3u);
            out[i] = s * (float)((lo | (hi << 4)) - 32);
        }
    } else {
        const u32x4 qv = realign(r.a, r.c, r.e);
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
        const float d = f16_to_f32(r.s);
#pragma unroll
        for (int i = 0; i < 16; i++) out[i] = d * (float)(int8_t)(q[i >> 2] >> (8 * (i & 3)));
    }
}

}  // namespace

template <uint32_t DT, int BM>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const uint8_t* __restrict__ W, int64_t rb, int N, int64_t K,
                                                       const float* __restrict__ x, int M,
                                                       const float* __restrict__ bias, float* __restrict__ y) {
    constexpr int TB = BM / 32;  // activation tiles of 16 per wave
    __shared__ __align__(16) float lw[2][GF_BN * GF_S];  // [buffer] weights [n][k]
    __shared__ __align__(16) float lx[2][BM * GF_S];     // [buffer] activations [m][k]
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n0 = blockIdx.x * GF_BN, m0 = blockIdx.y * BM;
    const int wn = (wave & 1) * 64, wm = (wave >> 1) * (BM / 2);
    // This thread's loads: row t/2 of each tile, k half t%2 (activations:
    // the threads of the first BM rows).
    const int lr = t >> 1, h = t & 1;
    const bool xload = lr < BM;
    const uint8_t* wrow = W + (int64_t)min(n0 + lr, N - 1) * rb;
    const float* xrow = x + (int64_t)min(m0 + min(lr, BM - 1), M - 1) * K + 16 * h;

    f32x4 acc[4][TB];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < TB; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto stage_store = [&](int buf, const WRaw& wr, const f32x4* xv, int64_t k0) {
        float wv[16];
        decode_w<DT>(wr, k0, wv);
        float* ws = &lw[buf][lr * GF_S + 16 * h];
#pragma unroll
        for (int i = 0; i < 8; i++) *(float2*)(ws + 2 * i) = float2{wv[2 * i], wv[2 * i + 1]};
        if (xload) {
            float* xs = &lx[buf][lr * GF_S + 16 * h];
#pragma unroll
            for (int i = 0; i < 8; i++)
                *(float2*)(xs + 2 * i) = float2{xv[i >> 1][2 * (i & 1)], xv[i >> 1][2 * (i & 1) + 1]};
        }
    };

    WRaw wr = load_w<DT>(wrow, 0, h);
    f32x4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) xv[i] = *(const f32x4*)(xrow + 4 * i);
    stage_store(0, wr, xv, 0);
    __syncthreads();

    const int nst = (int)(K / GF_BK);
    const int r16 = lane & 15, kq = lane >> 4;
    for (int s = 0; s < nst; s++) {
        const int buf = s & 1;
        const bool more = s + 1 < nst;
        const int64_t k1 = (int64_t)(s + 1) * GF_BK;
        if (more) {
            wr = load_w<DT>(wrow, k1, h);
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = *(const f32x4*)(xrow + k1 + 4 * i);
        }
        const float* ws = &lw[buf][0];
        const float* xs = &lx[buf][0];
#pragma unroll
        for (int k4 = 0; k4 < GF_BK / 4; k4++) {
            float av[4], bv[TB];
#pragma unroll
            for (int a = 0; a < 4; a++) av[a] = ws[(wn + 16 * a + r16) * GF_S + 4 * k4 + kq];
#pragma unroll
            for (int b = 0; b < TB; b++) bv[b] = xs[(wm + 16 * b + r16) * GF_S + 4 * k4 + kq];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < TB; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        if (more) stage_store(buf ^ 1, wr, xv, k1);
        __syncthreads();
    }

    // acc[a][b] lane l holds rows n = 16a + 4(l/16) + j (j = 0..3) of
    // activation row m = 16b + l%16, of this wave's quarter.
#pragma unroll
    for (int b = 0; b < TB; b++) {
        const int m = m0 + wm + 16 * b + r16;
        if (m >= M) continue;
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const int n = n0 + wn + 16 * a + 4 * kq;
            float* yr = y + (int64_t)m * N;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (n + j < N) {
                    float v = acc[a][b][j];
                    if (bias) v += bias[n + j];
                    yr[n + j] = v;
                }
            }
        }
    }
}

template <int BM>
static hipError_t launch_gf(const DevWeight& w, const float* x, int64_t rows, const float* bias, float* y,
                            hipStream_t stream) {
    dim3 grid((unsigned)((w.n + GF_BN - 1) / GF_BN), (unsigned)((rows + BM - 1) / BM)), blk(256);
    if (grid.y > 65535) return hipErrorInvalidValue;
    switch (w.dt) {
    case DT_Q4_K:
        hipLaunchKernelGGL((gemm_f32_kernel<DT_Q4_K, BM>), grid, blk, 0, stream, w.data, w.row_bytes, (int)w.n, w.k, x,
                           (int)rows, bias, y);
        break;
    case DT_Q6_K:
        hipLaunchKernelGGL((gemm_f32_kernel<DT_Q6_K, BM>), grid, blk, 0, stream, w.data, w.row_bytes, (int)w.n, w.k, x,
                           (int)rows, bias, y);
        break;
    case DT_Q8_0:
        hipLaunchKernelGGL((gemm_f32_kernel<DT_Q8_0, BM>), grid, blk, 0, stream, w.data, w.row_bytes, (int)w.n, w.k, x,
                           (int)rows, bias, y);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_linear_f32_mfma(const DevWeight& w, const float* x, int64_t rows, const float* bias, float* y,
                                  hipStream_t stream) {
    if (rows <= 0 || w.n <= 0) return hipSuccess;
    if (w.k % GF_BK || rows > INT32_MAX || w.n > INT32_MAX) return hipErrorInvalidValue;
    // 64-row tiles when 128-row tiles would not give every CU one.
    const int64_t tiles128 = (w.n + GF_BN - 1) / GF_BN * ((rows + 127) / 128);
    if (tiles128 < 256) return launch_gf<64>(w, x, rows, bias, y, stream);
    return launch_gf<128>(w, x, rows, bias, y, stream);
}

}  // namespace mimg
