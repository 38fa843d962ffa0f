// Prefill GEMM for small grids: Q4_K / Q6_K weights x 8-bit activations in
// blocks of 256 on v_mfma_i32_16x16x64_i8, 64 weight rows x 128 activation
// rows per workgroup of eight waves. gemm_kquant.hip's 32 x 32 x 32 kernel
// takes 128 x 128 tiles; where that gives fewer workgroups than the GPU has
// CUs (few weight rows or few activation rows, e.g. 64 prompt rows) this one
// runs instead. Same result, bit for bit (both equal the decode GEMV):
// per (weight row n, activation row m) and block b the exact int32
//   Q4_K  S = sum_k sc_s(k) q_k y_k,   M = sum_k m_s(k) y_k (= sum_s m_s xs_s)
//   Q6_K  S = sum_k sc_s(k) (q_k - 32) y_k
// then serially in block order tot = fma(f32(S), d*dx_b, tot) (and off for
// Q4_K), result tot - off (+ bias), as dotQ8KRef (reference
// internal/kernels/q8k_test.go:38-102; tiles as amx.go:194-316).
//
// Exact products on int8 MFMA: Q4_K sc = 8*sh + sl (sh, sl <= 7), planes
// sh*q and sl*q (each <= 105), S = 8*H + L; Q6_K w = 256*hi + lo, lo in
// [-128,127], hi in [-16,16]; Q4_K's M term is a third plane with A = m_s.
//
// Tiling (a shape C: T threads, NW waves along the weight rows, BM
// activation rows, NS stages): wave w takes weight rows 16(w % NW).. (A
// operand: lane l holds row l%16 and the 16 k of group l/16) against
// activation tiles of 16 (B, same k mapping); C lane l holds rows 4(l/16)+r,
// column l%16. Per block of 256 the raw weight blocks, the int8 activation
// rows and their scales are copied into LDS with global_load_lds, NS blocks
// in flight (a ring of NS stages). Activation rows sit in LDS with their
// 16-byte chunks XOR-swizzled by row (chunk c of row m at c ^ (m & 15)).
// Refused rows take the float32 path at the end.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {
namespace g16 {

typedef int v4i __attribute__((ext_vector_type(4)));

// A workgroup shape: T threads, NW waves along the weight rows (16 rows
// each), BM activation rows, NS stages in the copy ring.
template <int T_, int NW_, int BM_, int NS_>
struct GCfg {
    static constexpr int T = T_;          // threads per workgroup
    static constexpr int NW = NW_;        // waves along the weight rows
    static constexpr int BN = 16 * NW;    // weight rows per workgroup
    static constexpr int BM = BM_;        // activation rows per workgroup
    static constexpr int NS = NS_;        // blocks in flight
    static constexpr int WM = T / 64 / NW;    // waves along the activation rows
    static constexpr int TM = BM / 16 / WM;   // activation tiles of 16 per wave
    static constexpr int ACH = BM * 16 / T;   // activation copy instructions per thread per block
    static_assert(WM * NW * 64 == T && TM * WM * 16 == BM && T >= BN && T >= BM && ACH * T == BM * 16,
                  "GEMM tile shape");
};
// 64 weight rows x 128 activation rows, eight waves (large grids), and the
// shapes of few activation rows (up to 64): 32 or 16 weight rows, so that
// the grid holds as many workgroups as the GPU has CUs. The 32-row tiles
// take two waves, each its 16 weight rows against all 64 activation rows,
// so each weight plane is built once (gate at 64 rows 29.4 -> 27.7 us
// against four waves of 16 x 32).
using CfgWide = GCfg<512, 4, 128, 2>;
using CfgM64N32 = GCfg<128, 2, 64, 3>;
using CfgM64N16 = GCfg<256, 1, 64, 3>;

template <uint32_t DT, class C>
struct GemmLayout {
    // LDS bytes per weight row slot: Q4_K blocks are 16-byte aligned and
    // copied as 9 chunks; Q6_K blocks (2-byte aligned) are copied as the 54
    // aligned dwords that cover them.
    static constexpr int WSLOT = DT == DT_Q4_K ? 144 : 216;
    static constexpr int WDMA = DT == DT_Q4_K ? (C::BN * 9 + C::T - 1) / C::T   // copy instructions per
                                             : (C::BN * 54 + C::T - 1) / C::T;  // thread per block
    static constexpr int WBYTES = WDMA * C::T * (DT == DT_Q4_K ? 16 : 4);  // incl. slack for unconditional copies
    static constexpr int ABYTES = C::BM * 256;
    static constexpr int DXBYTES = C::T * 4;
    static constexpr int BUF = WBYTES + ABYTES + DXBYTES;
    static constexpr int NDMA = WDMA + C::ACH + 1;
    static_assert(C::NS * BUF <= 160 * 1024, "GEMM stages exceed LDS");
    static_assert((C::NS - 1) * NDMA < 64, "the ring's copies in flight exceed the wait counter");
};

struct GemmArgs {
    const uint8_t* W;
    const uint8_t* wref;   // [N]
    const float* bias;     // [N] or null
    float* y;              // [M][N]
    int64_t rb;            // bytes per weight row
    int N, M, nb;
    int64_t K;
    const int8_t* q;       // [M][K]
    const float* d32;      // [M][K/32]
    const int32_t* ok;     // [M]
    const float* x;        // [M][K] f32 (fallback)
    int fused;             // float32 fallback order (rows of the whole call <= 8)
};

// Global -> LDS copies (global_load_lds: lane i of the wave writes its 16
// or 4 bytes at the wave's LDS base + 16i or 4i). Written as inline
// assembly so that the compiler does not track them: it would otherwise wait
// for every copy in flight (vmcnt(0)) before the first LDS read of a block,
// including the next block's prefetch. The waits are explicit instead
// (GM_WAIT_VMCNT), and the compiler's own waits can only be stronger, the
// counter retiring in order.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
__device__ __forceinline__ void lds_copy16(const void* g, uint8_t* lds_wave_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr(lds_wave_base))
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* g, uint8_t* lds_wave_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr(lds_wave_base))
                 : "memory", "m0");
}

// s_waitcnt with vmcnt <= n (n < 64) and the other counters unconstrained.
#define GM_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
// s_waitcnt lgkmcnt(0) (LDS reads of this wave done).
#define GM_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// A workgroup barrier without the memory fence of __syncthreads, whose
// vmcnt(0) would also wait for the next block's copies in flight; the
// waits it needs are written out before it.
__device__ __forceinline__ void gm_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Issues the copies of block b into LDS buffer `buf` (every thread issues
// exactly NDMA instructions, so the wait counts are the same in each wave).
template <uint32_t DT, class C>
__device__ __forceinline__ void gemm_issue_block(const GemmArgs& A, int n0, int m0, int b, uint8_t* buf) {
    using L = GemmLayout<DT, C>;
    const int t = threadIdx.x, wave = t >> 6;  // wave of the workgroup (0 .. T/64-1)
    uint8_t* wl = buf;
    uint8_t* al = buf + L::WBYTES;
    uint8_t* dl = al + L::ABYTES;
    if constexpr (DT == DT_Q4_K) {
#pragma unroll
        for (int i = 0; i < L::WDMA; i++) {
            const int c = min(C::T * i + t, C::BN * 9 - 1);  // chunk of 16 bytes
            const int r = c / 9, j = c - 9 * r;
            const int n = min(n0 + r, A.N - 1);
            lds_copy16(A.W + (int64_t)n * A.rb + (int64_t)b * Q4K_BYTES + 16 * j, wl + 16 * (C::T * i + 64 * wave));
        }
    } else {
#pragma unroll
        for (int i = 0; i < L::WDMA; i++) {
            const int c = min(C::T * i + t, C::BN * 54 - 1);  // dword
            const int r = c / 54, j = c - 54 * r;
            const int n = min(n0 + r, A.N - 1);
            const uint8_t* blk = A.W + (int64_t)n * A.rb + (int64_t)b * Q6K_BYTES;
            const uint8_t* base = (const uint8_t*)__builtin_align_down(blk, 4);
            lds_copy4(base + 4 * j, wl + 4 * (C::T * i + 64 * wave));
        }
    }
#pragma unroll
    for (int i = 0; i < C::ACH; i++) {
        const int c = C::T * i + t;              // LDS chunk: row c/16, slot c%16
        const int r = c >> 4, s = c & 15;
        const int m = min(m0 + r, A.M - 1);
        lds_copy16(A.q + (int64_t)m * A.K + 256 * b + 16 * (s ^ (r & 15)), al + 16 * (C::T * i + 64 * wave));
    }
    {
        const int m = min(m0 + min(t, C::BM - 1), A.M - 1);
        lds_copy4(A.d32 + (int64_t)m * (A.K / 32) + 8 * b, dl + 4 * (64 * wave));  // slots t >= BM are slack
    }
}

// A thread's copy sources for block 0, fixed over the blocks (block b adds
// b times the block size), and the wave index as a scalar, so that each
// block's copies cost one 64-bit add each (and the Q6_K realignment) and
// their LDS bases are scalar: gemm_issue_block's copies, in the same order
// to the same LDS bytes.
template <uint32_t DT, class C>
struct KsCopy {
    using L = GemmLayout<DT, C>;
    const uint8_t* w[L::WDMA];  // Q4_K: the chunk's bytes in block 0; Q6_K: the row's block 0
    uint32_t j4[L::WDMA];       // Q6_K: the dword within the aligned block
    const int8_t* a[C::ACH];
    const float* dx;
    int wave;
    __device__ KsCopy(const GemmArgs& A, int n0, int m0) {
        const int t = threadIdx.x;
        wave = __builtin_amdgcn_readfirstlane(t >> 6);
#pragma unroll
        for (int i = 0; i < L::WDMA; i++) {
            if constexpr (DT == DT_Q4_K) {
                const int c = min(C::T * i + t, C::BN * 9 - 1);
                const int r = c / 9, j = c - 9 * r;
                w[i] = A.W + (int64_t)min(n0 + r, A.N - 1) * A.rb + 16 * j;
                j4[i] = 0;
            } else {
                const int c = min(C::T * i + t, C::BN * 54 - 1);
                const int r = c / 54, j = c - 54 * r;
                w[i] = A.W + (int64_t)min(n0 + r, A.N - 1) * A.rb;
                j4[i] = 4 * j;
            }
        }
#pragma unroll
        for (int i = 0; i < C::ACH; i++) {
            const int c = C::T * i + t;
            const int r = c >> 4, s = c & 15;
            a[i] = A.q + (int64_t)min(m0 + r, A.M - 1) * A.K + 16 * (s ^ (r & 15));
        }
        dx = A.d32 + (int64_t)min(m0 + min(t, C::BM - 1), A.M - 1) * (A.K / 32);
    }
    __device__ __forceinline__ void issue(int b, uint8_t* buf) const {
        uint8_t* wl = buf;
        uint8_t* al = buf + L::WBYTES;
        uint8_t* dl = al + L::ABYTES;
#pragma unroll
        for (int i = 0; i < L::WDMA; i++) {
            if constexpr (DT == DT_Q4_K) {
                lds_copy16(w[i] + (uint32_t)(b * Q4K_BYTES), wl + 16 * (C::T * i + 64 * wave));
            } else {
                const uint8_t* blk = w[i] + (uint32_t)(b * Q6K_BYTES);
                lds_copy4((const uint8_t*)__builtin_align_down(blk, 4) + j4[i], wl + 4 * (C::T * i + 64 * wave));
            }
        }
#pragma unroll
        for (int i = 0; i < C::ACH; i++) lds_copy16(a[i] + (uint32_t)(256 * b), al + 16 * (C::T * i + 64 * wave));
        lds_copy4(dx + 8 * b, dl + 4 * (64 * wave));  // slots t >= BM are slack
    }
};

// The A operands of k step ks (64 k) for this lane's weight row wr (the
// block in LDS) and k group G. Q4_K: sc = 8*sh + sl with sh, sl <= 7: sh*q
// and sl*q (q <= 15) are at most 105, so each plane is the packed nibbles
// times a small constant (16-bit lanes, no carry between the bytes); aM
// holds the sub-block's min m_s in every byte.
__device__ __forceinline__ void q4k_operands(const uint8_t* wr, const Q4KScales& s, int ks, int G, v4i& aH, v4i& aL,
                                             v4i& aM) {
    const int sub = 2 * ks + (G >> 1);
    const uint32_t sc = byte_of(s.sc, sub), mm = byte_of(s.m, sub);
    const u32x4 qraw = *(const u32x4*)(wr + 16 + 32 * ks + 16 * (G & 1));
    const uint32_t qd[4] = {qraw.x, qraw.y, qraw.z, qraw.w};
    const short sh = (short)(sc >> 3), sl = (short)(sc & 7);
    const s16x2 shp = {sh, sh}, slp = {sl, sl};
    const int shift = 4 * (G >> 1);  // low nibbles for G < 2, high for G >= 2
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const s16x2 nib = as_s16x2((qd[k] >> shift) & 0x0F0F0F0Fu);
        aH[k] = (int)as_u32(nib * shp);
        aL[k] = (int)as_u32(nib * slp);
        aM[k] = (int)(mm * 0x01010101u);
    }
}

// Q6_K: the two planes of sc*(q - 32) (hi and lo, S = 256 hi + lo) of k step
// ks for the block at wr (rsh = wr & 3, wra the dword below it).
__device__ __forceinline__ void q6k_operands(const uint32_t* wra, uint32_t rsh, const uint8_t* wr, int ks, int G,
                                             v4i& aH, v4i& aL) {
    auto rd16 = [&](int off) -> u32x4 {  // 16 bytes at wr + off (off % 4 == 0)
        const uint32_t* p = wra + off / 4;
        return u32x4{__builtin_amdgcn_alignbyte(p[1], p[0], rsh), __builtin_amdgcn_alignbyte(p[2], p[1], rsh),
                     __builtin_amdgcn_alignbyte(p[3], p[2], rsh), __builtin_amdgcn_alignbyte(p[4], p[3], rsh)};
    };
    const int h = ks >> 1, p = 2 * (ks & 1) + (G >> 1);
    const u32x4 ql = rd16(64 * h + 32 * (p & 1) + 16 * (G & 1));
    const u32x4 qh = rd16(128 + 32 * h + 16 * (G & 1));
    const int sc = (int)(int8_t)wr[192 + 8 * h + (G & 1) + 2 * p];
    // u = sc*q - 32*sc + 128 = w + 128 in 16-bit lanes (packed integer
    // multiply-add, exact: |u| <= 4224); hi = u's high byte, lo = w's low
    // byte = u's with the top bit flipped, so w = 256 hi + lo
    const short cu = (short)(128 - 32 * sc);
    const s16x2 sc2 = {(short)sc, (short)sc}, c2 = {cu, cu};
    const uint32_t qld[4] = {ql.x, ql.y, ql.z, ql.w}, qhd[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t q6 = (((p >> 1) ? (qld[k] >> 4) : qld[k]) & 0x0F0F0F0Fu) |
                            (((qhd[k] >> (2 * p)) & 0x03030303u) << 4);
        // bytes 0, 2 (ue) and 1, 3 (uo) of q6 as 16-bit lanes (selector 0x0C: a zero byte)
        const uint32_t ue = as_u32(as_s16x2(__builtin_amdgcn_perm(0u, q6, 0x0C020C00u)) * sc2 + c2);
        const uint32_t uo = as_u32(as_s16x2(__builtin_amdgcn_perm(0u, q6, 0x0C030C01u)) * sc2 + c2);
        // v_perm selector [src1.bX, src0.bX, src1.bY, src0.bY]: w0 w1 w2 w3
        aH[k] = (int)__builtin_amdgcn_perm(uo, ue, 0x07030501u);
        aL[k] = (int)(__builtin_amdgcn_perm(uo, ue, 0x06020400u) ^ 0x80808080u);
    }
}

template <uint32_t DT, class C>
__global__ __launch_bounds__(C::T) void gemm_a8k_kernel(GemmArgs A) {
    using L = GemmLayout<DT, C>;
    constexpr int GM_NW = C::NW, GM_BN = C::BN, GM_BM = C::BM, GM_TM = C::TM, GM_T = C::T, NS = C::NS;
    __shared__ __align__(16) uint8_t smem[NS * L::BUF];
    __shared__ int flags[2];
    const int t = threadIdx.x, l = t & 63;
    const int wn = (t >> 6) % GM_NW, wm = (t >> 6) / GM_NW;  // this wave's weight rows 16wn.., activation tiles wm*GM_TM..
    const int ar = l & 15, G = l >> 4;
    const int n0 = blockIdx.x * GM_BN, m0 = blockIdx.y * GM_BM;
    const int nb = A.nb;

    // Refusals of this tile: any weight row with a non-finite block scale,
    // any refused activation row.
    if (t == 0) flags[0] = 0;
    __syncthreads();
    {
        int f = 0;
        if (t < GM_BN && n0 + t < A.N) f |= A.wref[n0 + t] != 0;
        if (t < GM_BM && m0 + t < A.M) f |= A.ok[m0 + t] == 0;
        if (f) flags[0] = 1;
    }

    v4i accH[GM_TM], accL[GM_TM], accM[GM_TM];
    float tot[GM_TM][4], off[GM_TM][4];
#pragma unroll
    for (int mt = 0; mt < GM_TM; mt++) {
        accH[mt] = v4i{0, 0, 0, 0};
        accL[mt] = v4i{0, 0, 0, 0};
        accM[mt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < 4; r++) tot[mt][r] = off[mt][r] = 0.f;
    }

    // The ring: blocks 0 .. NS-2 first; at block b, block b + NS - 1 goes
    // into the stage block b - 1 used (every wave is past it: the barrier
    // that ends block b - 1). Past the last block the last one is copied
    // again into the free stage, so every thread always has the same
    // number of copies in flight and one wait count serves every block.
    const KsCopy<DT, C> cp(A, n0, m0);
#pragma unroll
    for (int i = 0; i < NS - 1; i++) cp.issue(min(i, nb - 1), smem + i * L::BUF);
    for (int b = 0; b < nb; b++) {
        uint8_t* buf = smem + (b % NS) * L::BUF;
        cp.issue(min(b + NS - 1, nb - 1), smem + ((b + NS - 1) % NS) * L::BUF);
        GM_WAIT_VMCNT((NS - 1) * L::NDMA);  // block b's copies (issued NS - 1 blocks earlier) have landed
        gm_barrier();
        const uint8_t* wl = buf;
        const uint8_t* al = buf + L::WBYTES;
        const float* dl = (const float*)(al + L::ABYTES);

        // A operand row (weights): wave rows 16*wave + ar.
        float dC[4], dminC[4];
        if constexpr (DT == DT_Q4_K) {
            const uint8_t* wr = wl + (16 * wn + ar) * L::WSLOT;
            const uint32_t* sw = (const uint32_t*)(wr + 4);
            const Q4KScales s = q4k_scales(sw[0], sw[1], sw[2]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t dd = *(const uint32_t*)(wl + (16 * wn + 4 * G + r) * L::WSLOT);
                dC[r] = f16_to_f32(dd & 0xFFFFu);
                dminC[r] = f16_to_f32(dd >> 16);
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                // All B operands of this k step first: their LDS latency then
                // hides under the unpacking of the A planes.
                v4i bvs[GM_TM];
#pragma unroll
                for (int mt = 0; mt < GM_TM; mt++) {
                    const int row = 16 * (wm * GM_TM + mt) + ar;
                    bvs[mt] = *(const v4i*)(al + row * 256 + 16 * ((4 * ks + G) ^ (row & 15)));
                }
                v4i aH, aL, aM;
                q4k_operands(wr, s, ks, G, aH, aL, aM);
#pragma unroll
                for (int mt = 0; mt < GM_TM; mt++) {
                    accH[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, bvs[mt], accH[mt], 0, 0, 0);
                    accL[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, bvs[mt], accL[mt], 0, 0, 0);
                    accM[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aM, bvs[mt], accM[mt], 0, 0, 0);
                }
            }
        } else {
            // Q6_K: the row's block starts sh bytes into its slot.
            auto wbyte_addr = [&](int row) -> const uint8_t* {
                const int n = min(n0 + row, A.N - 1);
                const uint8_t* blk = A.W + (int64_t)n * A.rb + (int64_t)b * Q6K_BYTES;
                return wl + row * L::WSLOT + ((uintptr_t)blk & 3);
            };
            const uint8_t* wr = wbyte_addr(16 * wn + ar);
            const uint32_t rsh = (uint32_t)((uintptr_t)wr & 3);
            const uint32_t* wra = (const uint32_t*)(wr - rsh);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint8_t* wc = wbyte_addr(16 * wn + 4 * G + r);
                dC[r] = f16_to_f32((uint32_t)wc[208] | ((uint32_t)wc[209] << 8));
                dminC[r] = 0.f;
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                // All B operands of this k step first: their LDS latency then
                // hides under the unpacking of the A planes.
                v4i bvs[GM_TM];
#pragma unroll
                for (int mt = 0; mt < GM_TM; mt++) {
                    const int row = 16 * (wm * GM_TM + mt) + ar;
                    bvs[mt] = *(const v4i*)(al + row * 256 + 16 * ((4 * ks + G) ^ (row & 15)));
                }
                v4i aH, aL;
                q6k_operands(wra, rsh, wr, ks, G, aH, aL);
#pragma unroll
                for (int mt = 0; mt < GM_TM; mt++) {
                    accH[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, bvs[mt], accH[mt], 0, 0, 0);
                    accL[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, bvs[mt], accL[mt], 0, 0, 0);
                }
            }
        }

        // The block's float step, per output in block order.
#pragma unroll
        for (int mt = 0; mt < GM_TM; mt++) {
            const float dx = dl[16 * (wm * GM_TM + mt) + ar];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int S = (accH[mt][r] << (DT == DT_Q4_K ? 3 : 8)) + accL[mt][r];
                tot[mt][r] = __builtin_fmaf((float)S, dC[r] * dx, tot[mt][r]);
                if (DT == DT_Q4_K) off[mt][r] = __builtin_fmaf((float)accM[mt][r], dminC[r] * dx, off[mt][r]);
            }
            accH[mt] = v4i{0, 0, 0, 0};
            accL[mt] = v4i{0, 0, 0, 0};
            accM[mt] = v4i{0, 0, 0, 0};
        }
        GM_WAIT_LGKM0();
        gm_barrier();  // stage b % NS is reloaded in the next iteration
    }
    GM_WAIT_VMCNT(0);  // the ring's extra copies have landed before the workgroup's LDS is given back

    // Outputs: lane holds rows n = n0 + 16*wave + 4G + r of column m.
    const int nbase = n0 + 16 * wn + 4 * G;
    const int refused = flags[0];
#pragma unroll
    for (int mt = 0; mt < GM_TM; mt++) {
        const int m = m0 + 16 * (wm * GM_TM + mt) + ar;
        if (m >= A.M) continue;
        if (refused && A.ok[m] == 0) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int n = nbase + r;
            if (n >= A.N) continue;
            if (refused && A.wref[n] != 0) continue;
            float res = DT == DT_Q4_K ? tot[mt][r] - off[mt][r] : tot[mt][r];
            if (A.bias) res += A.bias[n];
            A.y[(int64_t)m * A.N + n] = res;
        }
    }
    if (!refused) return;
    // Refused pairs of the tile: the float32 path, one group of eight lanes
    // per (row, activation row).
    const int g = t >> 3;
    for (int pidx = g; pidx < GM_BN * GM_BM; pidx += GM_T / 8) {
        const int n = n0 + pidx % GM_BN, m = m0 + pidx / GM_BN;
        if (n >= A.N || m >= A.M) continue;
        if (A.wref[n] == 0 && A.ok[m] != 0) continue;
        float res = f32dot_g8<DT>(A.W + (int64_t)n * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[n];
        if ((t & 7) == 0) A.y[(int64_t)m * A.N + n] = res;
    }
}

// Up to 64 activation rows with few weight rows (down at 64 prompt rows:
// 4096 rows, 256 workgroups of 16): the four waves of a workgroup split each
// block's four k steps of 64 instead of the activation rows, so each weight
// plane is built once and feeds all four 16-row activation tiles. Each wave
// writes its exact partial sums (S; Q4_K also the M term) per (activation
// row, weight row) to an LDS table; after a barrier every thread adds the
// four partials of its four (weight row, activation row) pairs (exact
// integers, any order) and runs the block's float step, the same as the
// other kernels: the result is bit for bit theirs.
// The copy layout of these workgroups (gemm_issue_block): 16 weight rows,
// BM activation rows, 256 threads, a ring of NS stages (Q6_K four: its
// tables are half Q4_K's, and 64-row down grids leave a CU to one workgroup;
// Q4_K three, so its 64-row tables fit beside the ring).
template <int BM_, int NS_>
struct KsCfg {
    static constexpr int T = 256, NW = 1, BN = 16, BM = BM_, NS = NS_;
    static constexpr int ACH = BM * 16 / T;
    static_assert(ACH * T == BM * 16, "k-step-split tile shape");
};
constexpr int KS_RS = 20;  // table row stride in ints: 16 weight rows + 4 of padding (banks)

// BMK activation rows (64, or 32: twice the workgroups, two or three a CU,
// for grids of few weight rows).
template <uint32_t DT, int BMK>
__global__ __launch_bounds__(256) void gemm_a8k_ks_kernel(GemmArgs A) {
    using C = KsCfg<BMK, DT == DT_Q6_K ? 4 : 3>;
    using L = GemmLayout<DT, C>;
    constexpr int NS = C::NS, TMK = BMK / 16, PPT = BMK / 16;  // activation tiles; pairs a thread
    constexpr int TAB = 4 * BMK * KS_RS;  // ints per table: [k step][activation row][weight row]
    typedef int vP __attribute__((ext_vector_type(PPT)));
    __shared__ __align__(16) uint8_t smem[NS * L::BUF];
    __shared__ __align__(16) int tabS[2 * TAB];  // two tables: block b's partials while block b - 1's are read
    __shared__ __align__(16) int tabM[DT == DT_Q4_K ? 2 * TAB : 4];
    __shared__ int flags[2];
    const int t = threadIdx.x, l = t & 63, ks = t >> 6;  // this wave's k step of each block
    const int ar = l & 15, G = l >> 4;
    const int n0 = blockIdx.x * 16, m0 = blockIdx.y * BMK;
    const int nb = A.nb;
    // The float step's pairs of this thread: activation row mc, weight rows PPT ng .. PPT ng + PPT - 1.
    const int mc = t % BMK, ng = t / BMK;

    if (t == 0) flags[0] = 0;
    __syncthreads();
    {
        int f = 0;
        if (t < 16 && n0 + t < A.N) f |= A.wref[n0 + t] != 0;
        if (t < BMK && m0 + t < A.M) f |= A.ok[m0 + t] == 0;
        if (f) flags[0] = 1;
    }
    float tot[PPT], off[PPT];
#pragma unroll
    for (int r = 0; r < PPT; r++) tot[r] = off[r] = 0.f;
    // Q6_K: the byte offset mod 4 of block 0 of this lane's row and of the
    // float step's rows (a block is 210 bytes, 2 mod 4: block b's offset is
    // that + 2b mod 4).
    uint32_t wsh0 = 0, fsh0[PPT];
#pragma unroll
    for (int r = 0; r < PPT; r++) fsh0[r] = 0;
    if constexpr (DT == DT_Q6_K) {
        wsh0 = (uint32_t)(uintptr_t)(A.W + (int64_t)min(n0 + ar, A.N - 1) * A.rb) & 3u;
#pragma unroll
        for (int r = 0; r < PPT; r++)
            fsh0[r] = (uint32_t)(uintptr_t)(A.W + (int64_t)min(n0 + PPT * ng + r, A.N - 1) * A.rb) & 3u;
    }
    // The block scales of the float step's rows, read from a block's stage
    // while it is current and used one block later.
    float dP[PPT], dminP[PPT], dxP = 0.f;
#pragma unroll
    for (int r = 0; r < PPT; r++) dP[r] = dminP[r] = 0.f;

    // The float step of block bb from table bb % 2 (this thread's PPT pairs,
    // in block order) with the scales read while bb's stage was current.
    auto float_step = [&](int bb) {
        const int* tS = tabS + (bb & 1) * TAB;
        vP S = *(const vP*)(tS + mc * KS_RS + PPT * ng);
#pragma unroll
        for (int k2 = 1; k2 < 4; k2++) S += *(const vP*)(tS + (k2 * BMK + mc) * KS_RS + PPT * ng);
        vP M = {};
        if constexpr (DT == DT_Q4_K) {
            const int* tM = tabM + (bb & 1) * TAB;
            M = *(const vP*)(tM + mc * KS_RS + PPT * ng);
#pragma unroll
            for (int k2 = 1; k2 < 4; k2++) M += *(const vP*)(tM + (k2 * BMK + mc) * KS_RS + PPT * ng);
        }
#pragma unroll
        for (int r = 0; r < PPT; r++) {
            tot[r] = __builtin_fmaf((float)S[r], dP[r] * dxP, tot[r]);
            if (DT == DT_Q4_K) off[r] = __builtin_fmaf((float)M[r], dminP[r] * dxP, off[r]);
        }
    };

    // The ring as in gemm_a8k_kernel, with one barrier a block: at block b
    // the waves write b's partials to table b % 2 and then run the float
    // step of block b - 1 from the other table. After the barrier that
    // starts block b every wave has finished block b - 1 (its reads of stage
    // b - 1 and of table b % 2), so block b + NS - 1 goes into stage b - 1
    // and the partials of b into table b % 2; the scales the float step of b
    // needs are read into registers while stage b is current.
    const KsCopy<DT, C> cp(A, n0, m0);
#pragma unroll
    for (int i = 0; i < NS - 1; i++) cp.issue(min(i, nb - 1), smem + i * L::BUF);
    for (int b = 0; b < nb; b++) {
        uint8_t* buf = smem + (b % NS) * L::BUF;
        GM_WAIT_VMCNT((NS - 2) * L::NDMA);  // block b's copies have landed
        GM_WAIT_LGKM0();                     // this wave's table writes of block b - 1 are done
        gm_barrier();
        cp.issue(min(b + NS - 1, nb - 1), smem + ((b + NS - 1) % NS) * L::BUF);
        const uint8_t* wl = buf;
        const uint8_t* al = buf + L::WBYTES;

        // This wave's k step against the activation tiles.
        v4i accH[TMK], accL[TMK], accM[TMK];
        v4i bvs[TMK];
#pragma unroll
        for (int mt = 0; mt < TMK; mt++) {
            const int row = 16 * mt + ar;
            bvs[mt] = *(const v4i*)(al + row * 256 + 16 * ((4 * ks + G) ^ (row & 15)));
        }
        const v4i z = {0, 0, 0, 0};
        if constexpr (DT == DT_Q4_K) {
            const uint8_t* wr = wl + ar * L::WSLOT;
            const uint32_t* sw = (const uint32_t*)(wr + 4);
            const Q4KScales sq = q4k_scales(sw[0], sw[1], sw[2]);
            v4i aH, aL, aM;
            q4k_operands(wr, sq, ks, G, aH, aL, aM);
#pragma unroll
            for (int mt = 0; mt < TMK; mt++) {
                accH[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, bvs[mt], z, 0, 0, 0);
                accL[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, bvs[mt], z, 0, 0, 0);
                accM[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aM, bvs[mt], z, 0, 0, 0);
            }
        } else {
            const uint32_t bsh = (wsh0 + 2u * (uint32_t)b) & 3u;
            const uint8_t* wr = wl + ar * L::WSLOT + bsh;
            const uint32_t rsh = (uint32_t)((uintptr_t)wr & 3);
            const uint32_t* wra = (const uint32_t*)(wr - rsh);
            v4i aH, aL;
            q6k_operands(wra, rsh, wr, ks, G, aH, aL);
#pragma unroll
            for (int mt = 0; mt < TMK; mt++) {
                accH[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, bvs[mt], z, 0, 0, 0);
                accL[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, bvs[mt], z, 0, 0, 0);
            }
        }
        // The float step of block b - 1 (its table is complete since the
        // barrier) while the MFMAs of block b run.
        if (b > 0) float_step(b - 1);
        // Block b's scales for the float step of the next iteration.
        dxP = ((const float*)(al + L::ABYTES))[mc];
#pragma unroll
        for (int r = 0; r < PPT; r++) {
            const int row = PPT * ng + r;
            if constexpr (DT == DT_Q4_K) {
                const uint32_t dd = *(const uint32_t*)(wl + row * L::WSLOT);
                dP[r] = f16_to_f32(dd & 0xFFFFu);
                dminP[r] = f16_to_f32(dd >> 16);
            } else {
                // d at byte 208 of the block: an even offset in the slot
                const uint32_t at = (uint32_t)(row * L::WSLOT) + ((fsh0[r] + 2u * (uint32_t)b) & 3u) + 208u;
                const uint32_t dw = *(const uint32_t*)(wl + (at & ~3u));
                dP[r] = f16_to_f32(dw >> (8u * (at & 2u)));
            }
        }
        // Partial sums to table b % 2: lane holds weight rows 4G..4G+3 of
        // activation row 16 mt + ar.
        int* tS = tabS + (b & 1) * TAB;
        int* tM = tabM + (DT == DT_Q4_K ? (b & 1) * TAB : 0);
#pragma unroll
        for (int mt = 0; mt < TMK; mt++) {
            v4i S;
#pragma unroll
            for (int r = 0; r < 4; r++) S[r] = (accH[mt][r] << (DT == DT_Q4_K ? 3 : 8)) + accL[mt][r];
            const int at = (ks * BMK + 16 * mt + ar) * KS_RS + 4 * G;
            *(v4i*)(tS + at) = S;
            if constexpr (DT == DT_Q4_K) *(v4i*)(tM + at) = accM[mt];
        }
    }
    GM_WAIT_LGKM0();
    gm_barrier();
    float_step(nb - 1);
    GM_WAIT_VMCNT(0);  // the ring's extra copies have landed before the workgroup's LDS is given back

    const int m = m0 + mc;
    const int refused = flags[0];
    if (m < A.M && !(refused && A.ok[m] == 0)) {
#pragma unroll
        for (int r = 0; r < PPT; r++) {
            const int n = n0 + PPT * ng + r;
            if (n >= A.N) continue;
            if (refused && A.wref[n] != 0) continue;
            float res = DT == DT_Q4_K ? tot[r] - off[r] : tot[r];
            if (A.bias) res += A.bias[n];
            A.y[(int64_t)m * A.N + n] = res;
        }
    }
    if (!refused) return;
    const int g = t >> 3;
    for (int pidx = g; pidx < 16 * BMK; pidx += 256 / 8) {
        const int n = n0 + pidx % 16, mm = m0 + pidx / 16;
        if (n >= A.N || mm >= A.M) continue;
        if (A.wref[n] == 0 && A.ok[mm] != 0) continue;
        float res = f32dot_g8<DT>(A.W + (int64_t)n * A.rb, A.x + (int64_t)mm * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[n];
        if ((t & 7) == 0) A.y[(int64_t)mm * A.N + n] = res;
    }
}

}  // namespace g16

template <class C>
static hipError_t launch_g16(const g16::GemmArgs& A, uint32_t dt, int64_t n, int64_t rows, hipStream_t stream) {
    using namespace g16;
    const dim3 grid((unsigned)((n + C::BN - 1) / C::BN), (unsigned)((rows + C::BM - 1) / C::BM));
    if (dt == DT_Q4_K)
        hipLaunchKernelGGL((gemm_a8k_kernel<DT_Q4_K, C>), grid, dim3(C::T), 0, stream, A);
    else
        hipLaunchKernelGGL((gemm_a8k_kernel<DT_Q6_K, C>), grid, dim3(C::T), 0, stream, A);
    return hipGetLastError();
}

// The 16 x 16 x 64 form of the prefill GEMM (see the top of this file).
// Up to 64 activation rows: 64-row tiles, 32 weight rows a workgroup where
// that gives at least 256 workgroups, else 16; more rows: 64 x 128 tiles,
// or 32 x 64 tiles where those give fewer than 256 workgroups.
hipError_t launch_gemm_a8k_16(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                           const float* bias, float* y, hipStream_t stream) {
    using namespace g16;
    if (!gemm_a8k_ok(w) || rows <= 0 || rows > (1 << 30) || w.n > (1 << 30)) return hipErrorInvalidValue;
    GemmArgs A;
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
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    if (rows <= 64) {
        if ((w.n + 31) / 32 >= 256) return launch_g16<CfgM64N32>(A, w.dt, w.n, rows, stream);
        // 32-row tiles up to 32 rows (down at 32 rows: 51.5 against 61.4 us
        // with 64-row tiles), 64-row tiles above (62.4 against 65.7 us at 64
        // rows: the 32-row tiles read each weight twice)
        const dim3 grid((unsigned)((w.n + 15) / 16), 1);
        if (rows <= 32) {
            if (w.dt == DT_Q4_K) hipLaunchKernelGGL((gemm_a8k_ks_kernel<DT_Q4_K, 32>), grid, dim3(256), 0, stream, A);
            else hipLaunchKernelGGL((gemm_a8k_ks_kernel<DT_Q6_K, 32>), grid, dim3(256), 0, stream, A);
        } else {
            if (w.dt == DT_Q4_K) hipLaunchKernelGGL((gemm_a8k_ks_kernel<DT_Q4_K, 64>), grid, dim3(256), 0, stream, A);
            else hipLaunchKernelGGL((gemm_a8k_ks_kernel<DT_Q6_K, 64>), grid, dim3(256), 0, stream, A);
        }
        return hipGetLastError();
    }
    // More rows on few weight rows (a prompt's k and v, 1024 rows): where the
    // 64 x 128 tiles leave CUs idle, 32 x 64 tiles (measured on MI355X: the
    // 8B prompt of 512 rows 24.5 -> 23.3 ms; the same tiles for q, o and
    // down at 512 rows, 256 workgroups of 64 x 128, made it 25.6 ms, and
    // 16 x 64 tiles 33.0 ms)
    if ((w.n + 63) / 64 * ((rows + 127) / 128) < 256) return launch_g16<CfgM64N32>(A, w.dt, w.n, rows, stream);
    return launch_g16<CfgWide>(A, w.dt, w.n, rows, stream);
}

}  // namespace mimg
