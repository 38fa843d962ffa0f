// Prefill GEMM, Q4_K / Q6_K weights x 8-bit activations in blocks of 32
// (dequant_matmul_a8.v1, and .v2 with block = 32; reference
// interp/fast.go:246-379) for many activation rows, on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8): one MFMA k step of 32 is one activation block,
// so each weight byte is read once per tile of activation rows instead of
// once per eight rows (the lane-order GEMV).
//
// Numerics: the reference's block-32 kernels' per-block form (dotQ4KQ8AVX2,
// internal/kernels/kernels_amd64.s:428-597, dotQ6KQ8AVX2 :760-882) with one
// float chain where they keep eight SIMD lanes. Per (weight row n,
// activation row m), weight block b and its activation blocks j = 0..7 in
// order, with exact int32 sums
//   Q4_K  S_j = sc_j * sum_{k in j} q_k y_k
//   Q6_K  S_j = sc_{2j} * sum_{k in 2j} (q_k - 32) y_k + sc_{2j+1} * sum_{k in 2j+1} (q_k - 32) y_k
//         (the two sub-blocks of 16 of activation block j)
// the float steps are t = fma(f32(S_j), dx_j, t), then tot = fma(d, t, tot)
// per block; Q4_K also off = fma(dmin * f32(m_j), dbs_j, off) per j (dbs_j
// = dx_j * f32(sum_{k in j} y_k), the quantizer's block sums); the result
// is tot - off (Q4_K) or tot, plus the bias. This is not the reference's
// lane order, so it is a tolerance claim (the spec's dequant_matmul_a8
// bound, spec/stdlib.md:260-275), which a caller opts into; each row's
// result depends on that row alone. Rows of x the quantizer refused and
// weight rows with a non-finite block scale take the reference's float32
// path.
//
// Tiling: a workgroup of NW x WM waves owns 32 NW weight rows x 64 WM
// activation rows; a wave takes 32 weight rows (the MFMA column operand,
// decoded per activation block from the raw weight block in LDS) against two
// row tiles of 32 activation rows. Lane l of a 32 x 32 result holds weight
// row l % 32 and activation rows 8j + 4(l/32) + r. Per weight block (256
// elements) the raw weight bytes, the int8 activation rows (16-byte chunks
// XOR-swizzled by row) and the rows' eight dx (and dbs) are copied into LDS
// with global_load_lds, double-buffered.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {
namespace kq32 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int NW_, int WM_>
struct Cfg {
    static constexpr int NW = NW_, WM = WM_;
    static constexpr int T = 64 * NW * WM;
    static constexpr int BN = 32 * NW;  // weight rows
    static constexpr int BM = 64 * WM;  // activation rows
};
using CfgWide = Cfg<4, 2>;  // 128 x 128, eight waves
using CfgMid = Cfg<2, 1>;   // 64 x 64, two waves

template <uint32_t DT, class C>
struct Lay {
    // 16-byte chunks of a weight row per block: Q4_K blocks are 16-byte
    // aligned (9 chunks); a Q6_K block (2-byte aligned) is covered by the 14
    // chunks from the 16-byte boundary below it.
    static constexpr int WCH = DT == DT_Q4_K ? 9 : 14;
    static constexpr int WSLOT = 16 * WCH;
    static constexpr int WDMA = (C::BN * WCH + C::T - 1) / C::T;
    static constexpr int WBYTES = WDMA * C::T * 16;  // incl. slack for unconditional copies
    static constexpr int ADMA = C::BM * 16 / C::T;
    static constexpr int ABYTES = C::BM * 256;
    static constexpr int XDMA = C::BM * 8 / C::T;   // dword copies of dx, [j][activation row]
    static constexpr int XBYTES = C::BM * 8 * 4;
    static constexpr int YDMA = DT == DT_Q4_K ? XDMA : 0;  // and of dbs (Q4_K)
    static constexpr int YBYTES = DT == DT_Q4_K ? XBYTES : 0;
    static constexpr int BUF = WBYTES + ABYTES + XBYTES + YBYTES;
    static constexpr int NDMA = WDMA + ADMA + XDMA + YDMA;
    static_assert(ADMA * C::T == C::BM * 16 && XDMA * C::T == C::BM * 8, "block-32 GEMM tile shape");
    static_assert(2 * BUF <= 160 * 1024 && NDMA < 64, "block-32 GEMM buffers");
};

struct Args {
    const uint8_t* W;
    const uint8_t* wref;   // [N]
    const float* bias;     // [N] or null
    float* y;              // [M][N]
    int64_t rb;            // bytes per weight row
    int N, M, nb;          // weight blocks per row
    int64_t K;
    const int8_t* q;       // [M][K]
    const float* d32;      // [M][K/32]
    const float* dbs;      // [M][K/32]
    const int32_t* ok;     // [M]
    const float* x;        // [M][K] f32 (fallback)
    int fused;
    int tiles_m;
};

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
// global_load_lds copies (lane i writes its bytes at the wave's LDS base +
// 16i or 4i), written as inline assembly so that the compiler does not wait
// for them at every LDS read; the waits are explicit.
__device__ __forceinline__ void lds_copy16(const void* g, uint8_t* lds_wave_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr(lds_wave_base))
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* g, uint8_t* lds_wave_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr(lds_wave_base))
                 : "memory", "m0");
}
#define KQ_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define KQ_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)
__device__ __forceinline__ void kq_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The start of weight row n's block b (global memory).
template <uint32_t DT>
__device__ __forceinline__ const uint8_t* wblock(const Args& A, int n, int b) {
    return A.W + (int64_t)n * A.rb + (int64_t)b * (DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES);
}

// The copies of weight block b into `buf` (every thread issues NDMA instructions).
template <uint32_t DT, class C>
__device__ __forceinline__ void issue_block(const Args& A, int n0, int m0, int b, uint8_t* buf) {
    using L = Lay<DT, C>;
    const int t = threadIdx.x, wave = t >> 6;
    uint8_t* wl = buf;
    uint8_t* al = buf + L::WBYTES;
    uint8_t* xl = al + L::ABYTES;
#pragma unroll
    for (int i = 0; i < L::WDMA; i++) {
        const int c = min(C::T * i + t, C::BN * L::WCH - 1);
        const int r = c / L::WCH, j = c - L::WCH * r;
        const int n = min(n0 + r, A.N - 1);
        const uint8_t* src = (const uint8_t*)__builtin_align_down(wblock<DT>(A, n, b), 16) + 16 * j;
        lds_copy16(src, wl + 16 * (C::T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < L::ADMA; i++) {
        const int c = C::T * i + t;  // row c/16, chunk c%16 stored at slot (c%16) ^ (row & 15)
        const int r = c >> 4, s = c & 15;
        const int m = min(m0 + r, A.M - 1);
        lds_copy16(A.q + (int64_t)m * A.K + 256 * b + 16 * (s ^ (r & 15)), al + 16 * (C::T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < L::XDMA; i++) {
        const int c = C::T * i + t;  // activation block j = c / BM, row c % BM
        const int j = c / C::BM, r = c - C::BM * j;
        const int m = min(m0 + r, A.M - 1);
        lds_copy4(A.d32 + (int64_t)m * (A.K / 32) + 8 * b + j, xl + 4 * (C::T * i + 64 * wave));
        if constexpr (DT == DT_Q4_K)
            lds_copy4(A.dbs + (int64_t)m * (A.K / 32) + 8 * b + j, xl + L::XBYTES + 4 * (C::T * i + 64 * wave));
    }
}

// 16 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ uint32_t lds_dw_a2(const uint8_t* p, int i) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    return __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}
__device__ __forceinline__ v4i lds_read16_a2(const uint8_t* p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
    return v4i{(int)__builtin_amdgcn_alignbyte(w1, w0, sh), (int)__builtin_amdgcn_alignbyte(w2, w1, sh),
               (int)__builtin_amdgcn_alignbyte(w3, w2, sh), (int)__builtin_amdgcn_alignbyte(w4, w3, sh)};
}

template <uint32_t DT, class C>
__global__ __launch_bounds__(C::T) void gemm_kq_b32_kernel(Args A) {
    using L = Lay<DT, C>;
    __shared__ __align__(16) uint8_t smem[2 * L::BUF];
    __shared__ int flags[1];
    const int t = threadIdx.x, l = t & 63, wave = t >> 6;
    const int wn = wave % C::NW, wm = wave / C::NW;
    const int a = l & 31, g = l >> 5;
    const int ntn = (A.N + C::BN - 1) / C::BN;
    const int nwg = ntn * A.tiles_m;
    int wg = blockIdx.x;
    if (nwg % 8 == 0) wg = (wg % 8) * (nwg / 8) + wg / 8;  // the row tiles of a weight tile on one XCD
    const int tile_n = wg / A.tiles_m, tile_m = wg % A.tiles_m;
    const int n0 = tile_n * C::BN, m0 = tile_m * C::BM;

    if (t == 0) flags[0] = 0;
    __syncthreads();
    {
        int f = 0;
        for (int i = t; i < C::BN || i < C::BM; i += C::T) {
            if (i < C::BN && n0 + i < A.N) f |= A.wref[n0 + i] != 0;
            if (i < C::BM && m0 + i < A.M) f |= A.ok[m0 + i] == 0;
        }
        if (f) flags[0] = 1;
    }

    // This lane's weight row (global, for the Q6_K block offsets).
    const int nrow = min(n0 + 32 * wn + a, A.N - 1);
    float tot[2][16], tb[2][16], off[2][16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        tot[0][i] = tot[1][i] = 0.f;
        tb[0][i] = tb[1][i] = 0.f;
        off[0][i] = off[1][i] = 0.f;
    }

    issue_block<DT, C>(A, n0, m0, 0, smem);
    for (int b = 0; b < A.nb; b++) {
        uint8_t* buf = smem + (b & 1) * L::BUF;
        if (b + 1 < A.nb) {
            issue_block<DT, C>(A, n0, m0, b + 1, smem + ((b + 1) & 1) * L::BUF);
            KQ_WAIT_VMCNT(L::NDMA);
        } else {
            KQ_WAIT_VMCNT(0);
        }
        kq_barrier();
        const uint8_t* al = buf + L::WBYTES;
        const float* xl = (const float*)(al + L::ABYTES);
        const float* yl = xl + C::BM * 8;
        // This lane's block (its row's bytes in the weight slot).
        const uint8_t* wr = buf + (32 * wn + a) * L::WSLOT;
        float d;
        if constexpr (DT == DT_Q4_K) {
            const uint32_t* w4 = (const uint32_t*)wr;
            const uint32_t dd = w4[0];
            d = f16_to_f32(dd & 0xFFFFu);
            const float dmin = f16_to_f32(dd >> 16);
            const Q4KScales s = q4k_scales(w4[1], w4[2], w4[3]);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const v4i raw = *(const v4i*)(wr + 16 + 32 * (j >> 1) + 16 * g);
                const int sh = 4 * (j & 1);
                const v4i bw = (raw >> sh) & 0x0F0F0F0F;
                const int sc = (int)byte_of(s.sc, j);
                const float dm = dmin * (float)byte_of(s.m, j);
                const v16i z = {};
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const int row = 64 * wm + 32 * tt + a;
                    const v4i av = *(const v4i*)(al + row * 256 + 16 * ((2 * j + g) ^ (row & 15)));
                    const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bw, z, 0, 0, 0);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int mrow = 64 * wm + 32 * tt + 8 * jj + 4 * g;
                        const float4 dx4 = *(const float4*)(xl + C::BM * j + mrow);
                        const float4 db4 = *(const float4*)(yl + C::BM * j + mrow);
                        const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
                        const float dbr[4] = {db4.x, db4.y, db4.z, db4.w};
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int S = __mul24(sc, P[4 * jj + r]);
                            tb[tt][4 * jj + r] = __builtin_fmaf((float)S, dxr[r], tb[tt][4 * jj + r]);
                            off[tt][4 * jj + r] = __builtin_fmaf(dm, dbr[r], off[tt][4 * jj + r]);
                        }
                    }
                }
            }
        } else {
            // Q6_K: ql at +0, qh at +128, scales at +192, d at +208 from the
            // block's start, sh bytes into the slot.
            const uint32_t sh = (uint32_t)((uintptr_t)wblock<DT>(A, nrow, b) & 15);
            const uint8_t* wq = wr + sh;
            d = f16_to_f32(lds_dw_a2(wq + 208, 0) & 0xFFFFu);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int hn = j >> 2, seg = j & 3;
                const v4i ql = lds_read16_a2(wq + 64 * hn + 32 * (seg & 1) + 16 * g);
                const v4i qh = lds_read16_a2(wq + 128 + 32 * hn + 16 * g);
                const v4i v = ((ql >> (4 * (seg >> 1))) & 0x0F0F0F0F) | (((qh >> (2 * seg)) & 0x03030303) << 4);
                // q - 32 in each byte (q <= 63): set the top bit, subtract 32
                // (no borrow between bytes), flip the top bit back
                const v4i w = ((v | (int)0x80808080) - 0x20202020) ^ (int)0x80808080;
                const v4i zero = {0, 0, 0, 0};
                const v4i w0 = g == 0 ? w : zero, w1 = g == 0 ? zero : w;  // sub-block 2j (k < 16) and 2j+1
                const uint32_t sw = lds_dw_a2(wq + 192 + 8 * hn + 2 * seg, 0);  // the two scales (and two more)
                const int sa = (int)(int8_t)(sw & 0xFFu), sb = (int)(int8_t)((sw >> 8) & 0xFFu);
                const v16i z = {};
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const int row = 64 * wm + 32 * tt + a;
                    const v4i av = *(const v4i*)(al + row * 256 + 16 * ((2 * j + g) ^ (row & 15)));
                    const v16i Pa = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, w0, z, 0, 0, 0);
                    const v16i Pb = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, w1, z, 0, 0, 0);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int mrow = 64 * wm + 32 * tt + 8 * jj + 4 * g;
                        const float4 dx4 = *(const float4*)(xl + C::BM * j + mrow);
                        const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int S = __mul24(sa, Pa[4 * jj + r]) +
                                          __mul24(sb, Pb[4 * jj + r]);
                            tb[tt][4 * jj + r] = __builtin_fmaf((float)S, dxr[r], tb[tt][4 * jj + r]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                tot[tt][i] = __builtin_fmaf(d, tb[tt][i], tot[tt][i]);
                tb[tt][i] = 0.f;
            }
        }
        KQ_WAIT_LGKM0();
        kq_barrier();  // buffer b & 1 is reloaded in the next iteration
    }

    const int n = n0 + 32 * wn + a;
    const int refused = flags[0];
    if (n < A.N && !(refused && A.wref[n] != 0)) {
        const float bn = A.bias ? A.bias[n] : 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + 64 * wm + 32 * tt + 8 * (i >> 2) + 4 * g + (i & 3);
                if (m >= A.M) continue;
                if (refused && A.ok[m] == 0) continue;
                float res = DT == DT_Q4_K ? tot[tt][i] - off[tt][i] : tot[tt][i];
                if (A.bias) res += bn;
                A.y[(int64_t)m * A.N + n] = res;
            }
        }
    }
    if (!refused) return;
    // Refused pairs of the tile: the reference's float32 path.
    const int grp = t >> 3;
    for (int pidx = grp; pidx < C::BN * C::BM; pidx += C::T / 8) {
        const int nn = n0 + pidx % C::BN, m = m0 + pidx / C::BN;
        if (nn >= A.N || m >= A.M) continue;
        if (A.wref[nn] == 0 && A.ok[m] != 0) continue;
        float res = f32dot_g8<DT>(A.W + (int64_t)nn * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[nn];
        if ((t & 7) == 0) A.y[(int64_t)m * A.N + nn] = res;
    }
}

template <class C>
static hipError_t launch_cfg(Args A, uint32_t dt, int64_t n, int64_t rows, hipStream_t stream) {
    A.tiles_m = (int)((rows + C::BM - 1) / C::BM);
    const int64_t nwg = (n + C::BN - 1) / C::BN * A.tiles_m;
    if (nwg > 0x7fffffff) return hipErrorInvalidValue;
    if (dt == DT_Q4_K)
        hipLaunchKernelGGL((gemm_kq_b32_kernel<DT_Q4_K, C>), dim3((unsigned)nwg), dim3(C::T), 0, stream, A);
    else
        hipLaunchKernelGGL((gemm_kq_b32_kernel<DT_Q6_K, C>), dim3((unsigned)nwg), dim3(C::T), 0, stream, A);
    return hipGetLastError();
}

template <class C>
static int64_t wgs(int64_t n, int64_t rows) {
    return (n + C::BN - 1) / C::BN * ((rows + C::BM - 1) / C::BM);
}

}  // namespace kq32

bool gemm_kq_b32_ok(const DevWeight& w) {
    return (w.dt == DT_Q4_K || w.dt == DT_Q6_K) && w.k % 256 == 0 && w.k > 0;
}

// The largest tile that still gives every CU a workgroup (256 on MI355X);
// up to 64 rows (or where neither does) the 16 x 64 tiles of gemm_b32s.hip.
hipError_t launch_gemm_kq_b32(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                              const float* bias, float* y, hipStream_t stream) {
    using namespace kq32;
    if (!gemm_kq_b32_ok(w) || rows <= 0 || rows > (1 << 30) || w.n > (1 << 30)) return hipErrorInvalidValue;
    Args A;
    A.W = w.data;
    A.wref = w.wref;
    A.bias = bias;
    A.y = y;
    A.rb = w.row_bytes;
    A.N = (int)w.n;
    A.M = (int)rows;
    A.nb = (int)(w.k / 256);
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.dbs = a.dbs;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    A.tiles_m = 1;
    if (wgs<CfgWide>(w.n, rows) >= 256) return launch_cfg<CfgWide>(A, w.dt, w.n, rows, stream);
    if (rows > 64 && wgs<CfgMid>(w.n, rows) >= 256) return launch_cfg<CfgMid>(A, w.dt, w.n, rows, stream);
    return launch_gemm_b32_small(w, a, rows, total_rows, x, bias, y, stream);
}

}  // namespace mimg
