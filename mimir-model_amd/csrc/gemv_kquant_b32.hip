// Q4_K / Q6_K weights x 8-bit activations in blocks of 32
// (dequant_matmul_a8.v1, or v2 with block = 32), in the float order of the
// reference's block-32 kernels: lane l of a group of eight is SIMD lane l of
// dotQ4KQ8AVX2 (reference internal/kernels/kernels_amd64.s:428-597) or
// dotQ6KQ8AVX2 (:760-882), whose x4 variants (:598, :883) give the same bits.
// Each lane owns the four consecutive elements 4l..4l+3 of every run of 32;
// its integer sums are exact (v_dot4_i32_i8) and its float steps are, per
// block b,
//   Q4_K  A = fma(f32(sc_2c * lo_c), dx_{2c}, A), B = fma(f32(sc_2c+1 * hi_c), dx_{2c+1}, B)
//         for the four chunks c in order, tot = fma(d, A + B, tot),
//         off = fma(dmin * f32(m_l), dbs_l, off) (lane l owns sub-block l);
//   Q6_K  for (h, p) in order: v = sc * sum((q - 32) y), A or B (p even or
//         odd) = fma(f32(v), dx_{4h+p}, .), tot = fma(d, A + B, tot);
// and the eight lanes end in the reference HSUM of tot - off (Q4_K) or tot.
// The oracle restates these lane orders from the assembly text; no golden
// output of the reference pins them, so they are checked against it bit for
// bit and against the spec tolerance.
//
// Rows of W with a non-finite block scale and refused activation rows take
// the float32 path (reference interp/fast.go:323-377).
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

__device__ __forceinline__ float hsum_lanes8(float a) {
    const int lane = threadIdx.x & 63, base = lane & ~7, l = lane & 7;
    const float c = a + __shfl(a, base + ((l + 4) & 7));
    const float e = c + __shfl(c, base + ((l + 1) & 7));
    const float r = e + __shfl(e, base + ((l + 2) & 7));
    return __shfl(r, base);
}

struct B32Args {
    const uint8_t* W;
    int64_t rb;
    int N;
    int64_t K;
    const int8_t* q;       // [rows][K]
    const float* d32;      // [rows][K/32]
    const float* dbs;      // [rows][K/32]
    const int32_t* ok;     // [rows]
    const uint8_t* wref;   // [N]
    const float* x;        // [rows][K]
    const float* bias;
    float* y;
    int64_t y_stride;
    int fused;
};

// One group of eight lanes per weight row, M activation rows per launch.
template <uint32_t DT, int M>
__global__ __launch_bounds__(256) void gemv_kq_b32_kernel(B32Args A) {
    const int g = threadIdx.x >> 3, l = threadIdx.x & 7;
    const int row = blockIdx.x * 32 + g;
    const int rowc = row < A.N ? row : A.N - 1;
    const uint8_t* wrow = A.W + (int64_t)rowc * A.rb;
    const int64_t nb = A.K / 256, R32 = A.K / 32, K = A.K;
    float tot[M], off[M];
#pragma unroll
    for (int m = 0; m < M; m++) tot[m] = off[m] = 0.f;

    for (int64_t b = 0; b < nb; b++) {
        const int8_t* yb = A.q + 256 * b;
        if constexpr (DT == DT_Q4_K) {
            const uint8_t* blk = wrow + b * Q4K_BYTES;
            const u32x4 hdr = *(const u32x4*)blk;
            const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
            const Q4KScales s = q4k_scales(hdr.y, hdr.z, hdr.w);
            uint32_t qd[4];
#pragma unroll
            for (int c = 0; c < 4; c++) qd[c] = *(const uint32_t*)(blk + 16 + 32 * c + 4 * l);
            const float dm = dmin * (float)byte_of(s.m, l);
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float* dx = A.d32 + m * R32 + 8 * b;
                off[m] = __builtin_fmaf(dm, A.dbs[m * R32 + 8 * b + l], off[m]);
                float a = 0.f, bb = 0.f;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int8_t* yc = yb + m * K + 64 * c + 4 * l;
                    const int lo = sdot4(qd[c] & 0x0F0F0F0Fu, *(const uint32_t*)yc, 0);
                    const int hi = sdot4((qd[c] >> 4) & 0x0F0F0F0Fu, *(const uint32_t*)(yc + 32), 0);
                    a = __builtin_fmaf((float)((int)byte_of(s.sc, 2 * c) * lo), dx[2 * c], a);
                    bb = __builtin_fmaf((float)((int)byte_of(s.sc, 2 * c + 1) * hi), dx[2 * c + 1], bb);
                }
                tot[m] = __builtin_fmaf(d, a + bb, tot[m]);
            }
        } else {
            const uint8_t* blk = wrow + b * Q6K_BYTES;
            const float d = f16_to_f32(load_u16(blk + 208));
            uint32_t qlw[4], qhw[2];
#pragma unroll
            for (int j = 0; j < 4; j++) qlw[j] = load4_a2(blk + 64 * (j >> 1) + 32 * (j & 1) + 4 * l);
#pragma unroll
            for (int h = 0; h < 2; h++) qhw[h] = load4_a2(blk + 128 + 32 * h + 4 * l);
            int scv[8];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int p = 0; p < 4; p++) scv[4 * h + p] = (int)(int8_t)blk[192 + 8 * h + 2 * p + (l >> 2)];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float* dx = A.d32 + m * R32 + 8 * b;
                float a = 0.f, bb = 0.f;
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        const uint32_t q6 = ((qlw[2 * h + (p & 1)] >> (4 * (p >> 1))) & 0x0F0F0F0Fu) |
                                            (((qhw[h] >> (2 * p)) & 0x03030303u) << 4);
                        const uint32_t yv = *(const uint32_t*)(yb + m * K + 128 * h + 32 * p + 4 * l);
                        const int sq = sdot4(q6, yv, 0) - 32 * sdot4(0x01010101u, yv, 0);
                        const float v = (float)(scv[4 * h + p] * sq);
                        if (p % 2 == 0) a = __builtin_fmaf(v, dx[4 * h + p], a);
                        else bb = __builtin_fmaf(v, dx[4 * h + p], bb);
                    }
                tot[m] = __builtin_fmaf(d, a + bb, tot[m]);
            }
        }
    }
    const bool wok = A.wref[rowc] == 0;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float r;
        if (wok && A.ok[m]) r = hsum_lanes8(DT == DT_Q4_K ? tot[m] - off[m] : tot[m]);
        else r = f32dot_g8<DT>(wrow, A.x + (int64_t)m * K, K, A.fused != 0);
        if (A.bias) r += A.bias[rowc];
        if (l == 0 && row < A.N) A.y[(int64_t)m * A.y_stride + row] = r;
    }
}

template <uint32_t DT, int M>
static void launch_b32(const B32Args& A, hipStream_t stream) {
    dim3 grid((unsigned)((A.N + 31) / 32)), blk(256);
    hipLaunchKernelGGL((gemv_kq_b32_kernel<DT, M>), grid, blk, 0, stream, A);
}

template <uint32_t DT>
static void launch_b32_rows(const B32Args& A, int rows, hipStream_t stream) {
    switch (rows) {
    case 1: launch_b32<DT, 1>(A, stream); break;
    case 2: launch_b32<DT, 2>(A, stream); break;
    case 3: launch_b32<DT, 3>(A, stream); break;
    case 4: launch_b32<DT, 4>(A, stream); break;
    case 5: launch_b32<DT, 5>(A, stream); break;
    case 6: launch_b32<DT, 6>(A, stream); break;
    case 7: launch_b32<DT, 7>(A, stream); break;
    default: launch_b32<DT, 8>(A, stream); break;
    }
}

hipError_t launch_gemv_kq_a8_b32(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows,
                                 const float* x, const float* bias, float* y, int64_t y_stride,
                                 hipStream_t stream) {
    if ((w.dt != DT_Q4_K && w.dt != DT_Q6_K) || w.k % 256 || rows < 1 || rows > 8) return hipErrorInvalidValue;
    B32Args A;
    A.W = w.data;
    A.rb = w.row_bytes;
    A.N = (int)w.n;
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.dbs = a.dbs;
    A.ok = a.ok;
    A.wref = w.wref;
    A.x = x;
    A.bias = bias;
    A.y = y;
    A.y_stride = y_stride;
    A.fused = total_rows <= 8;
    if (w.dt == DT_Q4_K) launch_b32_rows<DT_Q4_K>(A, (int)rows, stream);
    else launch_b32_rows<DT_Q6_K>(A, (int)rows, stream);
    return hipGetLastError();
}

}  // namespace mimg
