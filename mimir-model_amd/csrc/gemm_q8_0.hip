// Prefill GEMM, Q8_0 weights x 8-bit activations in blocks of 32
// (dequant_matmul_a8.v1, and .v2 with block = 32; reference
// interp/fast.go:246-379) for many activation rows, on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8): one MFMA k step of 32 is one Q8_0 block.
//
// Per (weight row n, activation row m) and block j of 32 elements the sum
// S = sum_k w_k y_k is exact in int32 (|S| <= 32 * 127 * 127); then, in
// block order, tot = fma(f32(S), f32(d_j) * dx_j, tot), and the result is
// tot (+ bias). The reference's dotQ8_0Q8AVX2 (kernels_amd64.s:1007-1043)
// keeps eight float chains of four-element sums and adds them in a tree at
// the end; this kernel keeps one chain of exact block sums (the order
// dotQ8KRef uses for blocks of 256, q8k_test.go:38-102). The two differ in
// the last bits; both are within the spec's tolerance for dequant_matmul_a8
// (spec/stdlib.md:260-275), which the tests check against the exact product
// of the decoded weights. Rows of x the quantizer refused and weight rows
// with a non-finite block scale take the reference's float32 path.
//
// Tiling: a workgroup of eight waves owns 128 weight rows x 128 activation
// rows; a wave takes 32 weight rows (the MFMA column operand, read from the
// raw blocks in LDS) against two row tiles of 32 activation rows. Lane l of
// the 32 x 32 result holds weight row l % 32 and activation rows
// 8j + 4(l/32) + r. K runs in groups of eight blocks (256 elements): the
// weight rows' 272 bytes, the int8 activation rows and their 8 scales per
// row are copied into LDS with global_load_lds, double-buffered. Within a
// group each wave issues block j's MFMAs, then runs block j-1's float step
// while they execute.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {
namespace q80 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// A workgroup shape: NW waves along the weight rows (32 each), WM along the
// activation rows (64 each).
template <int NW_, int WM_>
struct Cfg {
    static constexpr int NW = NW_, WM = WM_;
    static constexpr int T = 64 * NW * WM;
    static constexpr int BN = 32 * NW;   // weight rows
    static constexpr int BM = 64 * WM;   // activation rows
    static constexpr int GB = 8;         // Q8_0 blocks per group (256 elements)
    static constexpr int WSLOT = GB * Q80_BYTES;           // 272 bytes of a row per group (17 chunks of 16)
    static constexpr int WCH = WSLOT / 16;
    static constexpr int WDMA = (BN * WCH + T - 1) / T;    // 16-byte copies per thread per group
    static constexpr int WBYTES = WDMA * T * 16;
    static constexpr int ADMA = BM * 16 / T;
    static constexpr int ABYTES = BM * 256;
    static constexpr int XDMA = BM * GB / T;               // dword copies of the activation scales
    static constexpr int XBYTES = BM * GB * 4;             // [block j][activation row], f32
    static constexpr int BUF = WBYTES + ABYTES + XBYTES;
    static constexpr int NDMA = WDMA + ADMA + XDMA;
    static_assert(ADMA * T == BM * 16 && XDMA * T == BM * GB, "Q8_0 GEMM tile shape");
    static_assert(2 * BUF <= 160 * 1024 && NDMA < 64, "Q8_0 GEMM buffers");
};
// 128 x 128 (eight waves) where that gives every CU a workgroup, else
// 64 x 64 (two waves) above 64 rows; otherwise the 16 x 64 tiles of
// gemm_b32s.hip (four waves).
using CfgWide = Cfg<4, 2>;
using CfgMid = Cfg<2, 1>;

struct Args {
    const uint8_t* W;
    const uint8_t* wref;   // [N]
    const float* bias;     // [N] or null
    float* y;              // [M][N]
    int64_t rb;            // bytes per weight row
    int N, M, ng;          // groups of 8 blocks
    int64_t K;
    const int8_t* q;       // [M][K]
    const float* d32;      // [M][K/32]
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
#define Q8_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define Q8_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)
__device__ __forceinline__ void q8_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The copies of group gi into `buf` (every thread issues NDMA instructions).
template <class C>
__device__ __forceinline__ void issue_group(const Args& A, int n0, int m0, int gi, uint8_t* buf) {
    constexpr int T = C::T, BN = C::BN, BM = C::BM, GB = C::GB, WSLOT = C::WSLOT, WCH = C::WCH, WDMA = C::WDMA,
                  WBYTES = C::WBYTES, ADMA = C::ADMA, ABYTES = C::ABYTES, XDMA = C::XDMA;
    const int t = threadIdx.x, wave = t >> 6;
    uint8_t* wl = buf;
    uint8_t* al = buf + WBYTES;
    uint8_t* xl = al + ABYTES;
#pragma unroll
    for (int i = 0; i < WDMA; i++) {
        const int c = min(T * i + t, BN * WCH - 1);
        const int r = c / WCH, j = c - WCH * r;
        const int n = min(n0 + r, A.N - 1);
        lds_copy16(A.W + (int64_t)n * A.rb + (int64_t)gi * WSLOT + 16 * j, wl + 16 * (T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < ADMA; i++) {
        const int c = T * i + t;  // row c/16, chunk c%16 stored at slot (c%16) ^ (row & 15)
        const int r = c >> 4, s = c & 15;
        const int m = min(m0 + r, A.M - 1);
        lds_copy16(A.q + (int64_t)m * A.K + 256 * gi + 16 * (s ^ (r & 15)), al + 16 * (T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < XDMA; i++) {
        const int c = T * i + t;  // block j = c / BM, activation row c % BM
        const int j = c / BM, r = c - BM * j;
        const int m = min(m0 + r, A.M - 1);
        lds_copy4(A.d32 + (int64_t)m * (A.K / 32) + GB * gi + j, xl + 4 * (T * i + 64 * wave));
    }
}

// 16 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ v4i lds_read16_a2(const uint8_t* p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
    return v4i{(int)__builtin_amdgcn_alignbyte(w1, w0, sh), (int)__builtin_amdgcn_alignbyte(w2, w1, sh),
               (int)__builtin_amdgcn_alignbyte(w3, w2, sh), (int)__builtin_amdgcn_alignbyte(w4, w3, sh)};
}

template <class C>
__global__ __launch_bounds__(C::T) void gemm_q8_0_kernel(Args A) {
    constexpr int T = C::T, NW = C::NW, BN = C::BN, BM = C::BM, GB = C::GB, WSLOT = C::WSLOT, WBYTES = C::WBYTES,
                  ABYTES = C::ABYTES, BUF = C::BUF, NDMA = C::NDMA;
    __shared__ __align__(16) uint8_t smem[2 * BUF];
    __shared__ int flags[1];
    const int t = threadIdx.x, l = t & 63, wave = t >> 6;
    const int wn = wave % NW, wm = wave / NW;
    const int a = l & 31, g = l >> 5;
    const int ntn = (A.N + BN - 1) / BN;
    const int nwg = ntn * A.tiles_m;
    int wg = blockIdx.x;
    if (nwg % 8 == 0) wg = (wg % 8) * (nwg / 8) + wg / 8;  // row tiles of a weight tile on one XCD
    const int tile_n = wg / A.tiles_m, tile_m = wg % A.tiles_m;
    const int n0 = tile_n * BN, m0 = tile_m * BM;

    if (t == 0) flags[0] = 0;
    __syncthreads();
    {
        int f = 0;
        if (t < BN && n0 + t < A.N) f |= A.wref[n0 + t] != 0;
        if (t < BM && m0 + t < A.M) f |= A.ok[m0 + t] == 0;
        if (f) flags[0] = 1;
    }

    float tot[2][16];
#pragma unroll
    for (int i = 0; i < 16; i++) tot[0][i] = tot[1][i] = 0.f;

    issue_group<C>(A, n0, m0, 0, smem);
    for (int gi = 0; gi < A.ng; gi++) {
        uint8_t* buf = smem + (gi & 1) * BUF;
        if (gi + 1 < A.ng) {
            issue_group<C>(A, n0, m0, gi + 1, smem + ((gi + 1) & 1) * BUF);
            Q8_WAIT_VMCNT(NDMA);
        } else {
            Q8_WAIT_VMCNT(0);
        }
        q8_barrier();
        const uint8_t* wr = buf + (32 * wn + a) * WSLOT;
        const uint8_t* al = buf + WBYTES;
        const float* xl = (const float*)(al + ABYTES);
        v16i S[2][2];
        float dw[2];
        // block j's sums; then block j-1's float step while they run
        auto chain = [&](int j, const v16i (&s)[2], float d) {
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float4 dx4 = *(const float4*)(xl + BM * j + 64 * wm + 32 * tt + 8 * jj + 4 * g);
                    const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        tot[tt][4 * jj + r] = __builtin_fmaf((float)s[tt][4 * jj + r], d * dxr[r], tot[tt][4 * jj + r]);
                }
            }
        };
#pragma unroll
        for (int j = 0; j < GB; j++) {
            const v4i bw = lds_read16_a2(wr + Q80_BYTES * j + 2 + 16 * g);
            const uint32_t* dp = (const uint32_t*)__builtin_align_down(wr + Q80_BYTES * j, 4);
            dw[j & 1] = f16_to_f32(__builtin_amdgcn_alignbyte(dp[1], dp[0], (uint32_t)((uintptr_t)(wr + Q80_BYTES * j) & 3)) &
                                   0xFFFFu);
            const v16i z = {};
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int row = 64 * wm + 32 * tt + a;
                const v4i av = *(const v4i*)(al + row * 256 + 16 * ((2 * j + g) ^ (row & 15)));
                S[j & 1][tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bw, z, 0, 0, 0);
            }
            if (j > 0) chain(j - 1, S[(j - 1) & 1], dw[(j - 1) & 1]);
        }
        chain(GB - 1, S[(GB - 1) & 1], dw[(GB - 1) & 1]);
        Q8_WAIT_LGKM0();
        q8_barrier();
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
                float res = tot[tt][i];
                if (A.bias) res += bn;
                A.y[(int64_t)m * A.N + n] = res;
            }
        }
    }
    if (!refused) return;
    // Refused pairs of the tile: the reference's float32 path.
    const int grp = t >> 3;
    for (int pidx = grp; pidx < BN * BM; pidx += T / 8) {
        const int nn = n0 + pidx % BN, m = m0 + pidx / BN;
        if (nn >= A.N || m >= A.M) continue;
        if (A.wref[nn] == 0 && A.ok[m] != 0) continue;
        float res = f32dot_g8<DT_Q8_0>(A.W + (int64_t)nn * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[nn];
        if ((t & 7) == 0) A.y[(int64_t)m * A.N + nn] = res;
    }
}

}  // namespace q80

bool gemm_q8_0_ok(const DevWeight& w) { return w.dt == DT_Q8_0 && w.k % 256 == 0 && w.k > 0; }

template <class C>
static hipError_t launch_q80(q80::Args A, int64_t n, int64_t rows, hipStream_t stream) {
    A.tiles_m = (int)((rows + C::BM - 1) / C::BM);
    const int64_t nwg = (n + C::BN - 1) / C::BN * A.tiles_m;
    if (nwg > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(q80::gemm_q8_0_kernel<C>, dim3((unsigned)nwg), dim3(C::T), 0, stream, A);
    return hipGetLastError();
}

template <class C>
static int64_t q80_wgs(int64_t n, int64_t rows) {
    return (n + C::BN - 1) / C::BN * ((rows + C::BM - 1) / C::BM);
}

hipError_t launch_gemm_q8_0(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                            const float* bias, float* y, hipStream_t stream) {
    using namespace q80;
    if (!gemm_q8_0_ok(w) || rows <= 0 || rows > (1 << 30) || w.n > (1 << 30)) return hipErrorInvalidValue;
    Args A;
    A.W = w.data;
    A.wref = w.wref;
    A.bias = bias;
    A.y = y;
    A.rb = w.row_bytes;
    A.N = (int)w.n;
    A.M = (int)rows;
    A.ng = (int)(w.k / 256);
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    A.tiles_m = 1;
    if (q80_wgs<CfgWide>(w.n, rows) >= 256) return launch_q80<CfgWide>(A, w.n, rows, stream);
    if (rows > 64 && q80_wgs<CfgMid>(w.n, rows) >= 256) return launch_q80<CfgMid>(A, w.n, rows, stream);
    return launch_gemm_b32_small(w, a, rows, total_rows, x, bias, y, stream);
}

}  // namespace mimg
