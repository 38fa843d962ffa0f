// Decode GEMV, Q4_K / Q6_K weights x 8-bit activations in blocks of 256
// (dequant_matmul_a8.v2 with block = 256, the path mim-import writes for
// K-quant weights, reference importer/llama.go:264-280).
//
// Numerics (reference dotQ8KRef, internal/kernels/q8k_test.go:38-102, which
// dotQ4KQ8KAVX2/dotQ6KQ8KAVX2 and the x4/AMX/VNNI/NEON kernels all equal
// bit for bit): per block b the exact int32 sums
//   Q4_K  S = sum_s sc_s * sum_{k in s} q_k y_k,   M = sum_s m_s * xs_s
//   Q6_K  S = sum_s sc_s * sum_{k in s} (q_k - 32) y_k
// then, serially in block order,
//   tot = fma(f32(S), d*dx_b, tot),  off = fma(f32(M), dmin*dx_b, off)
// and the result is tot - off (Q4_K) or tot (Q6_K), plus bias[j] if given.
// f32(S) is v_cvt_f32_i32 (round to nearest even), d*dx one f32 multiply,
// fma one v_fma_f32, and the file is built with -ffp-contract=off.
//
// Mapping: a group of 8 lanes owns one weight row; a 256-thread workgroup
// holds 32 groups (32 rows). For each block, lane l of the group loads 16
// bytes of the block's quants (128-bit, coalesced) and computes its part of
// S with v_dot4_i32_i8; the group sums the parts with three DPP steps
// (integer, so exact in any order); every lane of the group then runs the
// same serial float chain. The activation quants of up to 8 rows are staged
// in LDS in tiles of blocks.
//
// Rows of x the quantizer refused and rows of w with a non-finite block scale
// take the float32 path (reference linearA8, interp/fast.go:323-377), in the
// reference's AVX2 order (f32path.hpp).
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

struct GemvArgs {
    const uint8_t* W;
    int64_t rb;      // bytes per weight row
    int N;           // weight rows
    int nb;          // blocks of 256 per row
    int64_t K;
    const int8_t* q;      // activation quants of the launch's first row
    const float* d32;     // [rows][K/32]
    const int16_t* s16;   // Q4_K: xs [rows][K/32]; Q6_K: ys16 [rows][K/16]
    const int32_t* ok;    // [rows]
    const uint8_t* wref;  // [N]
    const float* x;       // f32 activations (fallback)
    const float* bias;    // [N] or null
    float* y;             // [rows][y_stride]
    int64_t y_stride;
    int tb;               // blocks per LDS tile
    int fused;            // float32 fallback order: total rows <= 8
};

template <uint32_t DT>
struct KQ {
    static constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    static constexpr int S16PB = DT == DT_Q4_K ? 8 : 16;  // s16 entries per block
};

template <uint32_t DT, int M>
__global__ __launch_bounds__(256) void gemv_a8k_kernel(GemvArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int S16PB = KQ<DT>::S16PB;
    const int tb = A.tb;
    int8_t* qt = (int8_t*)smem;                                   // [M][tb*256]
    float* dxt = (float*)(smem + (size_t)M * tb * 256);           // [M][tb]
    int16_t* st = (int16_t*)(smem + (size_t)M * tb * 260);        // [M][tb*S16PB]

    const int g = threadIdx.x >> 3, l = threadIdx.x & 7;
    const int row = blockIdx.x * 32 + g;
    const int rowc = row < A.N ? row : A.N - 1;
    const uint8_t* wrow = A.W + (int64_t)rowc * A.rb;
    const int64_t R32 = A.K / 32, R16 = A.K / 16;

    float tot[M], off[M];
    for (int m = 0; m < M; m++) tot[m] = off[m] = 0.f;

    for (int kt = 0; kt < A.nb; kt += tb) {
        const int tcount = min(tb, A.nb - kt);
        __syncthreads();
        // Stage the tile's activation quants, block scales and sums in LDS.
        for (int i = threadIdx.x; i < M * tcount * 16; i += 256) {
            int m = i / (tcount * 16), o = i - m * tcount * 16;
            *(u32x4*)(qt + (size_t)m * tb * 256 + 16 * o) =
                *(const u32x4*)(A.q + (int64_t)m * A.K + (int64_t)kt * 256 + 16 * o);
        }
        for (int i = threadIdx.x; i < M * tcount; i += 256) {
            int m = i / tcount, o = i - m * tcount;
            dxt[m * tb + o] = A.d32[(int64_t)m * R32 + 8 * (int64_t)(kt + o)];
        }
        for (int i = threadIdx.x; i < M * tcount * S16PB; i += 256) {
            int m = i / (tcount * S16PB), o = i - m * tcount * S16PB;
            const int64_t stride = DT == DT_Q4_K ? R32 : R16;
            st[m * tb * S16PB + o] = A.s16[(int64_t)m * stride + (int64_t)kt * S16PB + o];
        }
        __syncthreads();

        for (int bb = 0; bb < tcount; bb++) {
            const int b = kt + bb;
            if (DT == DT_Q4_K) {
                const uint8_t* blk = wrow + (int64_t)b * Q4K_BYTES;
                const u32x4 hdr = *(const u32x4*)blk;
                const u32x4 qv = *(const u32x4*)(blk + 16 + 16 * l);
                const Q4KScales s = q4k_scales(hdr.y, hdr.z, hdr.w);
                const int c = l >> 1, h = l & 1;
                const int scl = (int)byte_of(s.sc, 2 * c), sch = (int)byte_of(s.sc, 2 * c + 1);
                const int mm = (int)byte_of(s.m, l);
                const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
                uint32_t lo[4], hi[4];
                lo[0] = qv.x & 0x0F0F0F0Fu; hi[0] = (qv.x >> 4) & 0x0F0F0F0Fu;
                lo[1] = qv.y & 0x0F0F0F0Fu; hi[1] = (qv.y >> 4) & 0x0F0F0F0Fu;
                lo[2] = qv.z & 0x0F0F0F0Fu; hi[2] = (qv.z >> 4) & 0x0F0F0F0Fu;
                lo[3] = qv.w & 0x0F0F0F0Fu; hi[3] = (qv.w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const int8_t* yb = qt + (size_t)m * tb * 256 + bb * 256 + 64 * c + 16 * h;
                    const u32x4 ya = *(const u32x4*)yb;
                    const u32x4 yh = *(const u32x4*)(yb + 32);
                    int dl = sdot4(lo[0], ya.x, 0);
                    dl = sdot4(lo[1], ya.y, dl);
                    dl = sdot4(lo[2], ya.z, dl);
                    dl = sdot4(lo[3], ya.w, dl);
                    int dh = sdot4(hi[0], yh.x, 0);
                    dh = sdot4(hi[1], yh.y, dh);
                    dh = sdot4(hi[2], yh.z, dh);
                    dh = sdot4(hi[3], yh.w, dh);
                    int S = group8_sum(scl * dl + sch * dh);
                    int Mt = group8_sum(mm * (int)st[m * tb * 8 + bb * 8 + l]);
                    const float dx = dxt[m * tb + bb];
                    tot[m] = __builtin_fmaf((float)S, d * dx, tot[m]);
                    off[m] = __builtin_fmaf((float)Mt, dmin * dx, off[m]);
                }
            } else {
                const uint8_t* blk = wrow + (int64_t)b * Q6K_BYTES;
                const int h = l >> 2, p = l & 3, pp = p >> 1, p1 = p & 1;
                const u32x4 qlv = load16_a2(blk + 64 * h + 16 * p);
                const u32x4 qhv = load16_a2(blk + 128 + 32 * h + 16 * p1);
                const uint32_t sw0 = load4_a2(blk + 192 + 8 * h);
                const uint32_t sw1 = load4_a2(blk + 196 + 8 * h);
                const int idx = 2 * pp + p1;
                const int scl = (int)(int8_t)(sw0 >> (8 * idx)), sch = (int)(int8_t)(sw1 >> (8 * idx));
                const float d = f16_to_f32(load_u16(blk + 208));
                const int shL = 2 * pp, shH = 4 + 2 * pp;
                uint32_t vl[4], vh[4];
                const uint32_t qlw[4] = {qlv.x, qlv.y, qlv.z, qlv.w};
                const uint32_t qhw[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    vl[k] = (qlw[k] & 0x0F0F0F0Fu) | (((qhw[k] >> shL) & 0x03030303u) << 4);
                    vh[k] = ((qlw[k] >> 4) & 0x0F0F0F0Fu) | (((qhw[k] >> shH) & 0x03030303u) << 4);
                }
                const int eL = 32 * pp + 16 * p1 + 128 * h, eH = eL + 64;
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const int8_t* yb = qt + (size_t)m * tb * 256 + bb * 256;
                    const u32x4 ya = *(const u32x4*)(yb + eL);
                    const u32x4 yh = *(const u32x4*)(yb + eH);
                    int dl = sdot4(vl[0], ya.x, 0);
                    dl = sdot4(vl[1], ya.y, dl);
                    dl = sdot4(vl[2], ya.z, dl);
                    dl = sdot4(vl[3], ya.w, dl);
                    int dh = sdot4(vh[0], yh.x, 0);
                    dh = sdot4(vh[1], yh.y, dh);
                    dh = sdot4(vh[2], yh.z, dh);
                    dh = sdot4(vh[3], yh.w, dh);
                    const int16_t* ys = st + m * tb * 16 + bb * 16;
                    int S = group8_sum(scl * (dl - 32 * (int)ys[eL >> 4]) + sch * (dh - 32 * (int)ys[eH >> 4]));
                    tot[m] = __builtin_fmaf((float)S, d * dxt[m * tb + bb], tot[m]);
                }
            }
        }
    }

    const bool wok = A.wref[rowc] == 0;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float r;
        if (wok && A.ok[m]) {
            r = DT == DT_Q4_K ? tot[m] - off[m] : tot[m];
        } else {
            r = f32dot_g8<DT>(wrow, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        }
        if (A.bias) r += A.bias[rowc];
        if (l == 0 && row < A.N) A.y[(int64_t)m * A.y_stride + row] = r;
    }
}

template <uint32_t DT, int M>
static hipError_t launch_m(GemvArgs A, hipStream_t stream) {
    A.tb = min(A.nb, max(1, 128 / M));
    const size_t lds = (size_t)M * A.tb * (256 + 4 + 2 * KQ<DT>::S16PB);
    dim3 grid((unsigned)((A.N + 31) / 32)), blk(256);
    hipLaunchKernelGGL((gemv_a8k_kernel<DT, M>), grid, blk, lds, stream, A);
    return hipGetLastError();
}

template <uint32_t DT>
static hipError_t launch_dt(GemvArgs A, int rows, hipStream_t stream) {
    switch (rows) {
    case 1: return launch_m<DT, 1>(A, stream);
    case 2: return launch_m<DT, 2>(A, stream);
    case 3: return launch_m<DT, 3>(A, stream);
    case 4: return launch_m<DT, 4>(A, stream);
    case 5: return launch_m<DT, 5>(A, stream);
    case 6: return launch_m<DT, 6>(A, stream);
    case 7: return launch_m<DT, 7>(A, stream);
    case 8: return launch_m<DT, 8>(A, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_a8k(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows,
                           const float* x, const float* bias, float* y, int64_t y_stride,
                           hipStream_t stream) {
    if (rows < 1 || rows > 8 || w.n <= 0 || w.k % 256) return hipErrorInvalidValue;
    GemvArgs A;
    A.W = w.data;
    A.rb = w.row_bytes;
    A.N = (int)w.n;
    A.nb = (int)(w.k / 256);
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.s16 = w.dt == DT_Q4_K ? a.xs : a.ys16;
    A.ok = a.ok;
    A.wref = w.wref;
    A.x = x;
    A.bias = bias;
    A.y = y;
    A.y_stride = y_stride;
    A.tb = 0;
    A.fused = total_rows <= 8;
    if (w.dt == DT_Q4_K) return launch_dt<DT_Q4_K>(A, (int)rows, stream);
    if (w.dt == DT_Q6_K) return launch_dt<DT_Q6_K>(A, (int)rows, stream);
    return hipErrorInvalidValue;
}

}  // namespace mimg
