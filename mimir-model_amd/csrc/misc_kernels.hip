// Smaller kernels of the path: the per-row refusal scan of a weight, block
// decode (mim.Dequantize), the float32-activation product
// (dequant_matmul.v1), and the Q8_0 x 8-bit block-32 GEMV.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// wref[j] = 1 if a block scale of row j is not finite: the 8-bit kernels
// refuse such rows (reference RowDot.DotQ8, internal/kernels/q8.go:125-130;
// dotQ8KRef checks d and dmin of Q4_K, d of Q6_K and Q8_0).
__global__ void weight_refusals_kernel(uint32_t dt, const uint8_t* __restrict__ w, int64_t n,
                                       int64_t nblk, int64_t bbytes, uint8_t* __restrict__ wref) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const uint8_t* row = w + j * nblk * bbytes;
    uint8_t bad = 0;
    for (int64_t b = 0; b < nblk; b++) {
        const uint8_t* blk = row + b * bbytes;
        if (dt == DT_Q4_K) bad |= (uint8_t)(!f16_finite(load_u16(blk)) || !f16_finite(load_u16(blk + 2)));
        else if (dt == DT_Q6_K) bad |= (uint8_t)!f16_finite(load_u16(blk + 208));
        else bad |= (uint8_t)!f16_finite(load_u16(blk));
    }
    wref[j] = bad;
}

hipError_t launch_weight_refusals(uint32_t dt, const uint8_t* w, int64_t n, int64_t k, uint8_t* wref,
                                  hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t be = dt == DT_Q8_0 ? 32 : 256;
    int64_t bb = dt == DT_Q4_K ? Q4K_BYTES : dt == DT_Q6_K ? Q6K_BYTES : Q80_BYTES;
    hipLaunchKernelGGL(weight_refusals_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       dt, w, n, k / be, bb, wref);
    return hipGetLastError();
}

// Block decode, bit-exact with mim.Dequantize (reference quant.go:197-344).
template <uint32_t DT>
__global__ void dequantize_kernel(const uint8_t* __restrict__ src, int64_t n, float* __restrict__ dst) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x)
        dst[e] = decode_weight<DT>(src, e);
}

hipError_t launch_dequantize(uint32_t dt, const uint8_t* src, int64_t n, float* dst, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536)), blk(256);
    switch (dt) {
    case DT_Q4_K: hipLaunchKernelGGL(dequantize_kernel<DT_Q4_K>, grid, blk, 0, stream, src, n, dst); break;
    case DT_Q6_K: hipLaunchKernelGGL(dequantize_kernel<DT_Q6_K>, grid, blk, 0, stream, src, n, dst); break;
    case DT_Q8_0: hipLaunchKernelGGL(dequantize_kernel<DT_Q8_0>, grid, blk, 0, stream, src, n, dst); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// dequant_matmul.v1 (reference linearF32/linearCols, interp/fast.go:161-183):
// one group of eight lanes per (weight row j, activation row i), the product
// in the reference's float order (f32path.hpp), then s + bias[j].
template <uint32_t DT>
__global__ __launch_bounds__(256) void linear_f32_kernel(const uint8_t* __restrict__ W, int64_t rb,
                                                         int64_t N, int64_t K,
                                                         const float* __restrict__ x, int64_t rows,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ y) {
    const int64_t pair = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int64_t pc = pair < N * rows ? pair : N * rows - 1;
    const int64_t i = pc / N, j = pc - i * N;
    float r = f32dot_g8<DT>(W + j * rb, x + i * K, K, rows <= 8);
    if (bias) r += bias[j];
    if ((threadIdx.x & 7) == 0 && pair < N * rows) y[i * N + j] = r;
}

hipError_t launch_linear_f32(const DevWeight& w, const float* x, int64_t rows, const float* bias,
                             float* y, hipStream_t stream) {
    if (rows <= 0 || w.n <= 0) return hipSuccess;
    int64_t pairs = rows * w.n;
    dim3 grid((unsigned)((pairs + 31) / 32)), blk(256);
    switch (w.dt) {
    case DT_Q4_K:
        hipLaunchKernelGGL(linear_f32_kernel<DT_Q4_K>, grid, blk, 0, stream, w.data, w.row_bytes, w.n, w.k, x, rows, bias, y);
        break;
    case DT_Q6_K:
        hipLaunchKernelGGL(linear_f32_kernel<DT_Q6_K>, grid, blk, 0, stream, w.data, w.row_bytes, w.n, w.k, x, rows, bias, y);
        break;
    case DT_Q8_0:
        hipLaunchKernelGGL(linear_f32_kernel<DT_Q8_0>, grid, blk, 0, stream, w.data, w.row_bytes, w.n, w.k, x, rows, bias, y);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// HSUM1 of the reference (kernels_amd64.s:405-411) over the eight lanes of a
// group: ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)), returned in every lane.
__device__ __forceinline__ float hsum1_group8(float a) {
    const int lane = threadIdx.x & 63, base = lane & ~7, l = lane & 7;
    float c = a + __shfl(a, base + ((l + 4) & 7));
    float e = c + __shfl(c, base + ((l + 1) & 7));
    float r = e + __shfl(e, base + ((l + 2) & 7));
    return __shfl(r, base);
}

// Q8_0 x 8-bit activations in blocks of 32 (dequant_matmul_a8.v1), in the
// order of dotQ8_0Q8AVX2 (reference kernels_amd64.s:1003-1043): lane l of a
// group of eight is SIMD lane l; per block it forms the exact sum P of
// elements 4l..4l+3 (one v_dot4_i32_i8) and acc = fma(f32(P), f32(d_w*dx), acc)
// in block order; the group then sums its lanes with HSUM1.
template <int M>
__global__ __launch_bounds__(256) void gemv_q8_0_a8_kernel(const uint8_t* __restrict__ W, int64_t rb,
                                                           int N, int64_t K,
                                                           const int8_t* __restrict__ q,
                                                           const float* __restrict__ d32,
                                                           const int32_t* __restrict__ ok,
                                                           const uint8_t* __restrict__ wref,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ y, int64_t y_stride,
                                                           int fused) {
    const int g = threadIdx.x >> 3, l = threadIdx.x & 7;
    const int row = blockIdx.x * 32 + g;
    const int rowc = row < N ? row : N - 1;
    const uint8_t* wrow = W + (int64_t)rowc * rb;
    const int64_t nb = K / 32;
    float acc[M];
    for (int m = 0; m < M; m++) acc[m] = 0.f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t* blk = wrow + b * Q80_BYTES;
        const uint32_t wq = load4_a2(blk + 2 + 4 * l);
        const float dw = f16_to_f32(load_u16(blk));
#pragma unroll
        for (int m = 0; m < M; m++) {
            const uint32_t yq = *(const uint32_t*)(q + (int64_t)m * K + 32 * b + 4 * l);
            const int P = sdot4(wq, yq, 0);
            acc[m] = __builtin_fmaf((float)P, dw * d32[(int64_t)m * nb + b], acc[m]);
        }
    }
    const bool wok = wref[rowc] == 0;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float r;
        if (wok && ok[m]) r = hsum1_group8(acc[m]);
        else r = f32dot_g8<DT_Q8_0>(wrow, x + (int64_t)m * K, K, fused != 0);
        if (bias) r += bias[rowc];
        if (l == 0 && row < N) y[(int64_t)m * y_stride + row] = r;
    }
}

template <int M>
static void launch_q80(const DevWeight& w, const ActPtrs& a, const float* x, const float* bias, float* y,
                       int64_t y_stride, int fused, hipStream_t stream) {
    dim3 grid((unsigned)((w.n + 31) / 32)), blk(256);
    hipLaunchKernelGGL(gemv_q8_0_a8_kernel<M>, grid, blk, 0, stream, w.data, w.row_bytes, (int)w.n, w.k,
                       a.q, a.d32, a.ok, w.wref, x, bias, y, y_stride, fused);
}

hipError_t launch_gemv_q8_0_a8(const DevWeight& w, const ActPtrs& a, int64_t rows,
                               int64_t total_rows, const float* x, const float* bias, float* y,
                               int64_t y_stride, hipStream_t stream) {
    if (w.dt != DT_Q8_0 || w.k % 32 || rows < 1 || rows > 8) return hipErrorInvalidValue;
    int fused = total_rows <= 8;
    switch (rows) {
    case 1: launch_q80<1>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 2: launch_q80<2>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 3: launch_q80<3>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 4: launch_q80<4>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 5: launch_q80<5>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 6: launch_q80<6>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 7: launch_q80<7>(w, a, x, bias, y, y_stride, fused, stream); break;
    case 8: launch_q80<8>(w, a, x, bias, y, y_stride, fused, stream); break;
    }
    return hipGetLastError();
}

}  // namespace mimg

namespace mimg {

// Streaming read of up to three byte ranges, the measuring stick of the
// HBM-bound kernels: workgroup w reads PER*4 KB of one range with 16-byte
// nontemporal loads, all of a thread's loads issued before any is used, and
// folds them with XOR. A store that depends on every loaded value (taken
// only for one bit pattern that random weights never produce) keeps the
// loads, so the kernel writes nothing in practice.
template <int PER>
__global__ __launch_bounds__(256) void stream_read_kernel(ReadRanges r, uint32_t* __restrict__ sink) {
    int64_t wg = blockIdx.x;
    int i = 0;
    while (i + 1 < r.count && wg >= r.wgs[i]) wg -= r.wgs[i++];
    constexpr int64_t CHUNK = (int64_t)PER * 256 * 16;
    const int64_t off = wg * CHUNK;
    const int64_t n16 = (r.len[i] - off < CHUNK ? r.len[i] - off : CHUNK) / 16;
    const u32x4* p = (const u32x4*)(r.src[i] + off);
    u32x4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int64_t idx = threadIdx.x + 256 * k;
        v[k] = idx < n16 ? __builtin_nontemporal_load(p + idx) : u32x4{0, 0, 0, 0};
    }
    uint32_t x = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) x ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (x == 0x9E3779B9u) sink[blockIdx.x & 1023] = x;
}

hipError_t launch_stream_read(const ReadRanges& r0, int per, uint32_t* sink, hipStream_t s) {
    ReadRanges r = r0;
    const int64_t chunk = (int64_t)per * 256 * 16;
    int64_t total = 0;
    for (int i = 0; i < r.count; i++) total += (r.wgs[i] = (r.len[i] + chunk - 1) / chunk);
    if (total <= 0 || total > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)total);
    switch (per) {
    case 2: hipLaunchKernelGGL(stream_read_kernel<2>, grid, dim3(256), 0, s, r, sink); break;
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, grid, dim3(256), 0, s, r, sink); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, grid, dim3(256), 0, s, r, sink); break;
    case 16: hipLaunchKernelGGL(stream_read_kernel<16>, grid, dim3(256), 0, s, r, sink); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mimg
