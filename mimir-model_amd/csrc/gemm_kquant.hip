// Prefill GEMM, Q4_K / Q6_K weights x 8-bit activations in blocks of 256
// (dequant_matmul_a8.v2, block = 256) for many activation rows, on the int8
// matrix cores (v_mfma_i32_32x32x32_i8). The result equals the decode GEMV's
// bit for bit, as the reference's AMX/VNNI tile kernels equal its one-row
// kernel (reference internal/kernels/amx.go:194-316, amx_test.go:41-141):
// per (weight row n, activation row m) and block b the exact int32
//   Q4_K  S = sum_k sc_s(k) q_k y_k,   M = sum_k m_s(k) y_k (= sum_s m_s xs_s)
//   Q6_K  S = sum_k sc_s(k) (q_k - 32) y_k
// then serially in block order tot = fma(f32(S), d*dx_b, tot) (and off for
// Q4_K), result tot - off (+ bias), as dotQ8KRef (q8k_test.go:38-102).
//
// Exact integer products on int8 MFMA: the scaled weight w = sc*q does not
// fit int8 (Q4_K up to 945, Q6_K -4096..4064), so it is split in two planes.
// Q4_K: sc = 8*sh + sl (sh, sl <= 7), planes sh*q and sl*q (each <= 105),
// S = 8*sum(sh*q*y) + sum(sl*q*y); the planes are the packed nibbles times
// a constant. Q6_K: w = 256*hi + lo with lo the low byte of w as a signed
// value (-128..127) and hi in [-16, 16], S = 256*sum(hi*y) + sum(lo*y):
// with u = w + 128 in a 16-bit lane, hi is u's high byte and lo its low
// byte with the top bit flipped. Each MFMA sum is exact in int32 (|sum| <
// 2^31 for 256-element blocks). Q4_K's M term = sum_s m_s xs_s comes from
// the activation's per-32 sums xs: one v_mfma_f32_32x32x16_f16 a row tile
// and block, with xs split as 64 hi + lo so that every operand is an exact
// f16 and every partial sum an integer below 2^24 (measured on MI355X
// against a third int8 plane with operand m_s over the 256 k: gate
// M = 2048 525 -> 460 us, M = 512 122 -> 114 us).
//
// Operands: the activation rows are the MFMA's row operand and the weight
// rows its column operand, so a lane of the 32 x 32 result holds one weight
// row (lane l: row l % 32) and 16 activation rows (8j + 4(l/32) + r), and
// needs one block scale d (and dmin) per block. A k step of 32 is one
// sub-block; lane l supplies k 16(l/32)..+15 of it for both operands.
//
// Tiling: a workgroup of NW x WM waves owns 32 NW weight rows x 64 WM
// activation rows; a wave takes 32 weight rows (its column tile, unpacked
// in registers from the raw blocks) against two row tiles of 32 activation
// rows. Per block of 256 the raw weight blocks (as in the file), the int8
// activation rows and their scales are copied into LDS with
// global_load_lds, double-buffered: block b+1 loads while block b computes.
// Activation rows sit in LDS with their 16-byte chunks XOR-swizzled by row
// (chunk c of row m at c ^ (m & 15)): the 32 lanes of a row-operand read,
// one chunk of 32 consecutive rows, touch every bank once per 16 rows.
//
// Rows of x the quantizer refused and weight rows with a non-finite block
// scale take the float32 path (reference interp/fast.go:323-377) at the end.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Workgroup shape: NW waves along the weight rows (32 each), WM along the
// activation rows (64 each: two MFMA row tiles).
template <uint32_t DT, int NW, int WM>
struct GemmLayout {
    static constexpr int T = 64 * NW * WM;   // threads
    static constexpr int BN = 32 * NW;       // weight rows per workgroup
    static constexpr int BM = 64 * WM;       // activation rows per workgroup
    // LDS per weight row: a Q4_K block (16-byte aligned) as its 9 chunks of
    // 16 bytes; a Q6_K block (2-byte aligned) as the 14 aligned chunks that
    // cover it and one more, the block starting (address & 15) bytes into its
    // slot. The fifteenth chunk puts rows 60 dwords apart instead of 56: the
    // dword reads of 32 rows then meet each bank twice, not four times
    // (measured on MI355X: down M = 2048 509 -> 478 us).
    static constexpr int WCH = DT == DT_Q4_K ? 9 : 15;
    static constexpr int WSLOT = 16 * WCH;
    static constexpr int WDMA = (BN * WCH + T - 1) / T;  // copies per thread per block
    static constexpr int WBYTES = WDMA * T * 16;         // incl. slack for unconditional copies
    static constexpr int ADMA = BM * 16 / T;
    static constexpr int ABYTES = BM * 256;
    // Q4_K: the block's per-32 activation sums xs (eight int16, 16 bytes) of
    // the BM rows, one copy per thread of a group of 256 (slots past BM:
    // the last row again)
    static constexpr int XBYTES = DT == DT_Q4_K ? 256 * 16 : 0;
    static constexpr int BUF = WBYTES + ABYTES + XBYTES;
    static constexpr int DXBYTES = T * 4;                // one dword copy per thread (BM used)
    static_assert(ADMA * T == BM * 16 && T >= BM && BM <= 256 && WM == 2, "GEMM tile shape");
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
    const int16_t* xs;     // [M][K/32]
    const int32_t* ok;     // [M]
    const float* x;        // [M][K] f32 (fallback)
    int fused;             // float32 fallback order (rows of the whole call <= 8)
    int tiles_m;           // row tiles of BM activation rows
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

// Byte offset of block b of weight row n inside its LDS slot (Q6_K blocks
// are copied from the 16-byte boundary below them).
__device__ __forceinline__ uint32_t q6k_slot_off(const GemmArgs& A, int n, int b) {
    return (uint32_t)(((uint64_t)n * (uint64_t)A.rb + (uint64_t)b * Q6K_BYTES) & 15u);
}

// Issues the copies of block b into LDS buffer `buf` (every thread issues
// exactly NDMA instructions, so the wait counts are the same in each wave).
template <uint32_t DT, int NW, int WM>
__device__ __forceinline__ void gemm_issue_block(const GemmArgs& A, int n0, int m0, int b, uint8_t* buf, uint8_t* dl) {
    using L = GemmLayout<DT, NW, WM>;
    const int t = threadIdx.x, wave = t >> 6;
    uint8_t* wl = buf;
    uint8_t* al = buf + L::WBYTES;
#pragma unroll
    for (int i = 0; i < L::WDMA; i++) {
        const int c = min(L::T * i + t, L::BN * L::WCH - 1);  // chunk of 16 bytes
        const int r = c / L::WCH, j = c - L::WCH * r;
        const int n = min(n0 + r, A.N - 1);
        const uint8_t* blk = A.W + (int64_t)n * A.rb + (int64_t)b * (DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES);
        const uint8_t* base = DT == DT_Q4_K ? blk : (const uint8_t*)__builtin_align_down(blk, 16);
        lds_copy16(base + 16 * j, wl + 16 * (L::T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < L::ADMA; i++) {
        const int c = L::T * i + t;  // LDS chunk: row c/16, slot c%16
        const int r = c >> 4, s = c & 15;
        const int m = min(m0 + r, A.M - 1);
        lds_copy16(A.q + (int64_t)m * A.K + 256 * b + 16 * (s ^ (r & 15)), al + 16 * (L::T * i + 64 * wave));
    }
    {
        const int m = min(m0 + min(t, L::BM - 1), A.M - 1);
        lds_copy4(A.d32 + (int64_t)m * (A.K / 32) + 8 * b, dl + 4 * (64 * wave));  // slots t >= BM are slack
    }
    if constexpr (DT == DT_Q4_K) {
        if (wave < 4) {
            const int m = min(m0 + min(t, L::BM - 1), A.M - 1);
            lds_copy16(A.xs + (int64_t)m * (A.K / 32) + 8 * b, al + L::ABYTES + 16 * (64 * wave));
        }
    }
}

// The same copies issued by the four trailing waves only (rank tr of 256),
// during their half of the block that runs the float chain: the leading
// waves' half holds the MFMAs and must not wait behind copy issue (measured
// on MI355X at gate M = 2048: 4-7 % faster than every wave issuing its share).
template <uint32_t DT, int NW, int WM>
__device__ __forceinline__ void gemm_issue_block_tr(const GemmArgs& A, int n0, int m0, int b, uint8_t* buf, uint8_t* dl,
                                                    int tr) {
    using L = GemmLayout<DT, NW, WM>;
    constexpr int T2 = 256, WD2 = (L::BN * L::WCH + T2 - 1) / T2, AD2 = L::BM * 16 / T2;
    static_assert(WD2 * T2 * 16 <= L::WBYTES && L::BM <= T2, "trailer copy layout");
    const int wt = tr >> 6;
    uint8_t* wl = buf;
    uint8_t* al = buf + L::WBYTES;
#pragma unroll
    for (int i = 0; i < WD2; i++) {
        const int c = min(T2 * i + tr, L::BN * L::WCH - 1);
        const int r = c / L::WCH, j = c - L::WCH * r;
        const int n = min(n0 + r, A.N - 1);
        const uint8_t* blk = A.W + (int64_t)n * A.rb + (int64_t)b * (DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES);
        const uint8_t* base = DT == DT_Q4_K ? blk : (const uint8_t*)__builtin_align_down(blk, 16);
        lds_copy16(base + 16 * j, wl + 16 * (T2 * i + 64 * wt));
    }
#pragma unroll
    for (int i = 0; i < AD2; i++) {
        const int c = T2 * i + tr;
        const int r = c >> 4, s = c & 15;
        const int m = min(m0 + r, A.M - 1);
        lds_copy16(A.q + (int64_t)m * A.K + 256 * b + 16 * (s ^ (r & 15)), al + 16 * (T2 * i + 64 * wt));
    }
    {
        const int m = min(m0 + min(tr, L::BM - 1), A.M - 1);
        lds_copy4(A.d32 + (int64_t)m * (A.K / 32) + 8 * b, dl + 4 * (64 * wt));
    }
    if constexpr (DT == DT_Q4_K) {
        const int m = min(m0 + min(tr, L::BM - 1), A.M - 1);
        lds_copy16(A.xs + (int64_t)m * (A.K / 32) + 8 * b, al + L::ABYTES + 16 * (64 * wt));
    }
}

// 16 bytes at an LDS address that is 2-byte aligned: five aligned dwords
// and a byte realignment.
__device__ __forceinline__ u32x4 lds_read16_a2(const uint8_t* p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
    return u32x4{__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                 __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh)};
}

template <uint32_t DT, int NW, int WM>
__global__ __launch_bounds__(64 * NW * WM) void gemm_a8k_kernel(GemmArgs A) {
    using L = GemmLayout<DT, NW, WM>;
    __shared__ __align__(16) uint8_t smem[2 * L::BUF];
    __shared__ __align__(16) uint8_t dxs[3 * L::DXBYTES];
    __shared__ int flags[1];
    const int t = threadIdx.x, l = t & 63, wave = t >> 6;
    const int wn = wave % NW, wm = wave / NW;
    const int a = l & 31, g = l >> 5;
    // Workgroups are dealt to the XCDs in turn; consecutive row tiles of
    // one weight tile go to the same XCD (and its L2) where possible.
    const int ntn = (A.N + L::BN - 1) / L::BN;
    const int nwg = ntn * A.tiles_m;
    int wg = blockIdx.x;
    if (nwg % 8 == 0) wg = (wg % 8) * (nwg / 8) + wg / 8;
    const int tile_n = wg / A.tiles_m, tile_m = wg % A.tiles_m;
    const int n0 = tile_n * L::BN, m0 = tile_m * L::BM;
    const int nb = A.nb;
    const int nrow = min(n0 + 32 * wn + a, A.N - 1);  // this lane's weight row (clamped)
    // The two waves on a SIMD run half a block apart: while one issues block
    // b's MFMAs the other runs block b-1's float chain, and they swap at each
    // barrier, so the matrix core and the vector unit of the SIMD work at the
    // same time. Waves w and w ^ 4 share a SIMD when waves are dealt to the
    // SIMDs in turn, w and w ^ 1 when dealt in pairs: this split puts a
    // leader and a trailer on each SIMD either way.
    const bool leader = ((wave ^ (wave >> 2)) & 1) == 0;
    const int trank = ((wave == 1 ? 0 : wave == 3 ? 1 : wave == 4 ? 2 : 3) << 6) + l;  // trailers 1, 3, 4, 6

    // Refusals of this tile: any weight row with a non-finite block scale,
    // any refused activation row.
    if (t == 0) flags[0] = 0;
    __syncthreads();
    {
        int f = 0;
        if (t < L::BN && n0 + t < A.N) f |= A.wref[n0 + t] != 0;
        if (t < L::BM && m0 + t < A.M) f |= A.ok[m0 + t] == 0;
        if (f) flags[0] = 1;
    }

    float tot[2][16], off[2][16];
#pragma unroll
    for (int i = 0; i < 16; i++) tot[0][i] = tot[1][i] = off[0][i] = off[1][i] = 0.f;
    v16i accH[2], accL[2];
    v16f accM[2];  // Q4_K: the mins term, exact integers in f32
    float dN = 0.f, dminN = 0.f;

    // Block b's integer sums (the MFMAs) from LDS buffer b & 1.
    auto block_sums = [&](int b) {
        const uint8_t* buf = smem + (b & 1) * L::BUF;
        const uint8_t* wl = buf;
        const uint8_t* al = buf + L::WBYTES;
        // row operands of k step ks: 16 bytes of two activation rows
        auto arow = [&](int ks, int tt) -> v4i {
            const int row = 64 * wm + 32 * tt + a;
            return *(const v4i*)(al + row * 256 + 16 * ((2 * ks + g) ^ (row & 15)));
        };
        if constexpr (DT == DT_Q4_K) {
            const uint8_t* wr = wl + (32 * wn + a) * L::WSLOT;
            const uint32_t dd = *(const uint32_t*)wr;
            dN = f16_to_f32(dd & 0xFFFFu);
            dminN = f16_to_f32(dd >> 16);
            const uint32_t* sw = (const uint32_t*)(wr + 4);
            const Q4KScales s = q4k_scales(sw[0], sw[1], sw[2]);
            u32x4 qv[4];
#pragma unroll
            for (int c = 0; c < 4; c++) qv[c] = *(const u32x4*)(wr + 16 + 32 * c + 16 * g);
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const v4i a0 = arow(ks, 0), a1 = arow(ks, 1);
                const uint32_t sc = byte_of(s.sc, ks);
                // sc = 8*sh + sl with sh, sl <= 7: sh*q and sl*q (q <= 15) are at
                // most 105, so each plane is the packed nibbles times a small
                // constant (16-bit lanes, no carry between the bytes).
                const short sh = (short)(sc >> 3), sl = (short)(sc & 7);
                const s16x2 shp = {sh, sh}, slp = {sl, sl};
                const int shift = 4 * (ks & 1);  // sub-block 2c: low nibbles, 2c+1: high
                const u32x4 qd = qv[ks >> 1];
                v4i bH, bL;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const s16x2 nib = as_s16x2((qd[k] >> shift) & 0x0F0F0F0Fu);
                    bH[k] = (int)as_u32(nib * shp);
                    bL[k] = (int)as_u32(nib * slp);
                }
                const v16i z = {};
                accH[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bH, ks ? accH[0] : z, 0, 0, 0);
                accH[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bH, ks ? accH[1] : z, 0, 0, 0);
                accL[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bL, ks ? accL[0] : z, 0, 0, 0);
                accL[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bL, ks ? accL[1] : z, 0, 0, 0);
            }
            // The mins term M = sum_s m_s xs_s of every (weight row,
            // activation row) on one f16 MFMA a row tile (k = 16: the eight
            // sub-blocks twice). xs = 64 hi + lo with hi in [-64, 63] and lo
            // in [0, 63]: the row operand holds hi_s at k = s (lanes g = 0)
            // and lo_s at k = 8 + s (g = 1), the weight operand 64 m_s and
            // m_s. Every product and partial sum is an integer below 2^24,
            // so the f32 result is M exactly. The f16 values are built as
            // f16(1024 + v) from the bits 0x6400 + v, minus 1024.
            {
                const uint32_t mw[2] = {(uint32_t)s.m, (uint32_t)(s.m >> 32)};
                const h2 mul = g ? h2{(_Float16)1.0f, (_Float16)1.0f} : h2{(_Float16)64.0f, (_Float16)64.0f};
                const h2 c1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
                v8h bm;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t u = __builtin_amdgcn_perm(0u, mw[j >> 1], (j & 1) ? 0x0C030C02u : 0x0C010C00u);
                    const h2 f = (__builtin_bit_cast(h2, u | 0x64006400u) - c1024) * mul;
                    bm[2 * j] = f.x;
                    bm[2 * j + 1] = f.y;
                }
                const uint8_t* xl = al + L::ABYTES;
                const short sh = g ? 0 : 6;
                const s16x2 sh2 = {sh, sh};
                const uint32_t msk = g ? 0x003F003Fu : 0xFFFFFFFFu;
                const h2 cf = g ? c1024 : h2{(_Float16)1088.0f, (_Float16)1088.0f};
                const s16x2 cadd = g ? s16x2{0x6400, 0x6400} : s16x2{0x6440, 0x6440};
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const u32x4 xw = *(const u32x4*)(xl + 16 * (64 * wm + 32 * tt + a));
                    const uint32_t xd[4] = {xw.x, xw.y, xw.z, xw.w};
                    v8h av;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t v = as_u32(as_s16x2(xd[j]) >> sh2) & msk;
                        const h2 f = __builtin_bit_cast(h2, as_u32(as_s16x2(v) + cadd)) - cf;
                        av[2 * j] = f.x;
                        av[2 * j + 1] = f.y;
                    }
                    const v16f zf = {};
                    accM[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bm, zf, 0, 0, 0);
                }
            }
        } else {
            const uint8_t* wr = wl + (32 * wn + a) * L::WSLOT + q6k_slot_off(A, nrow, b);
            u32x4 qlv[4], qhv[2];
#pragma unroll
            for (int i = 0; i < 4; i++) qlv[i] = lds_read16_a2(wr + 64 * (i >> 1) + 32 * (i & 1) + 16 * g);
#pragma unroll
            for (int h = 0; h < 2; h++) qhv[h] = lds_read16_a2(wr + 128 + 32 * h + 16 * g);
            const u32x4 scv = lds_read16_a2(wr + 192);
            {
                const uint32_t* dw = (const uint32_t*)__builtin_align_down(wr + 208, 4);
                const uint32_t sh = (uint32_t)((uintptr_t)(wr + 208) & 3);
                dN = f16_to_f32(__builtin_amdgcn_alignbyte(dw[1], dw[0], sh) & 0xFFFFu);
            }
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const v4i a0 = arow(ks, 0), a1 = arow(ks, 1);
                const int h = ks >> 2, p = ks & 3;
                const u32x4 ql = qlv[2 * h + (p & 1)], qh = qhv[h];
                const int si = 8 * h + g + 2 * p;  // scale of this lane's 16 elements
                const int sc = (int)(int8_t)(uint8_t)(scv[si >> 2] >> (8 * (si & 3)));
                // u = sc*q - 32*sc + 128 = w + 128 in 16-bit lanes (packed
                // integer multiply-add, exact: |u| <= 4224)
                const short cu = (short)(128 - 32 * sc);
                const s16x2 sc2 = {(short)sc, (short)sc}, c2 = {cu, cu};
                v4i bH, bL;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t q6 = (((p >> 1) ? (ql[k] >> 4) : ql[k]) & 0x0F0F0F0Fu) |
                                        (((qh[k] >> (2 * p)) & 0x03030303u) << 4);
                    const uint32_t ue = as_u32(as_s16x2(__builtin_amdgcn_perm(0u, q6, 0x0C020C00u)) * sc2 + c2);
                    const uint32_t uo = as_u32(as_s16x2(__builtin_amdgcn_perm(0u, q6, 0x0C030C01u)) * sc2 + c2);
                    // v_perm selector [src1.bX, src0.bX, src1.bY, src0.bY]: the
                    // high bytes of the lanes (hi) and the low bytes (lo + 128)
                    bH[k] = (int)__builtin_amdgcn_perm(uo, ue, 0x07030501u);
                    bL[k] = (int)(__builtin_amdgcn_perm(uo, ue, 0x06020400u) ^ 0x80808080u);
                }
                const v16i z = {};
                accH[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bH, ks ? accH[0] : z, 0, 0, 0);
                accH[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bH, ks ? accH[1] : z, 0, 0, 0);
                accL[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bL, ks ? accL[0] : z, 0, 0, 0);
                accL[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bL, ks ? accL[1] : z, 0, 0, 0);
            }
        }
    };
    // Block b's float step, per output in block order: lane l holds
    // activation rows 8j + 4g + r of each row tile against its weight row.
    auto block_chain = [&](int b) {
        const float* dl = (const float*)(dxs + (b % 3) * L::DXBYTES);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 dx4 = *(const float4*)(dl + 64 * wm + 32 * tt + 8 * j + 4 * g);
                const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = 4 * j + r;
                    const int S = (accH[tt][i] << (DT == DT_Q4_K ? 3 : 8)) + accL[tt][i];
                    tot[tt][i] = __builtin_fmaf((float)S, dN * dxr[r], tot[tt][i]);
                    if constexpr (DT == DT_Q4_K) off[tt][i] = __builtin_fmaf(accM[tt][i], dminN * dxr[r], off[tt][i]);
                }
            }
        }
    };

    // Block b's copies (weights and activations into buffer b & 1, the
    // activation scales into dx stage b % 3) are issued by the trailing waves
    // at the start of the first half of block b-1 and waited for at the end
    // of its second half.
    // Buffer (b+1) & 1 was last read by the trailing waves' sums of block
    // b-1, before the barrier that starts block b's first half; dx stage
    // (b+1) % 3 by the chain of block b-2.
    gemm_issue_block<DT, NW, WM>(A, n0, m0, 0, smem, dxs);
    GM_WAIT_VMCNT(0);
    gm_barrier();
    for (int b = 0; b <= nb; b++) {
        // first half: the leaders' sums of block b, the trailers' chain of b-1
        if (b + 1 < nb && !leader)
            gemm_issue_block_tr<DT, NW, WM>(A, n0, m0, b + 1, smem + ((b + 1) & 1) * L::BUF,
                                            dxs + ((b + 1) % 3) * L::DXBYTES, trank);
        if (leader) {
            if (b < nb) block_sums(b);
        } else if (b > 0) {
            block_chain(b - 1);
        }
        GM_WAIT_LGKM0();
        gm_barrier();
        if (b == nb) break;
        // second half: the leaders' chain of block b, the trailers' sums of b
        if (leader) block_chain(b);
        else block_sums(b);
        GM_WAIT_VMCNT(0);  // block b+1's copies have landed
        GM_WAIT_LGKM0();
        gm_barrier();
    }

    // Outputs: lane l holds weight row n against activation rows m.
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
    // Refused pairs of the tile: the float32 path, one group of eight lanes
    // per (row, activation row).
    const int grp = t >> 3;
    for (int pidx = grp; pidx < L::BN * L::BM; pidx += L::T / 8) {
        const int nn = n0 + pidx % L::BN, m = m0 + pidx / L::BN;
        if (nn >= A.N || m >= A.M) continue;
        if (A.wref[nn] == 0 && A.ok[m] != 0) continue;
        float res = f32dot_g8<DT>(A.W + (int64_t)nn * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[nn];
        if ((t & 7) == 0) A.y[(int64_t)m * A.N + nn] = res;
    }
}

bool gemm_a8k_ok(const DevWeight& w) {
    return (w.dt == DT_Q4_K || w.dt == DT_Q6_K) && w.k % 256 == 0 && w.k > 0;
}

hipError_t launch_gemm_a8k(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                           const float* bias, float* y, hipStream_t stream) {
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
    A.xs = a.xs;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    // 128 weight rows x 128 activation rows per workgroup of eight waves;
    // where that leaves CUs without a workgroup (few weight or activation
    // rows: down at 512 rows, 64 prompt rows) the 16 x 16 x 64 kernel with
    // 64-row tiles runs instead (measured on MI355X: gate/down at 64 rows
    // 41/155 against 57/218 us, down at 512 rows 176 against 222 us).
    constexpr int BN = 128, BM = 128;
    A.tiles_m = (int)((rows + BM - 1) / BM);
    const int64_t nwg = (w.n + BN - 1) / BN * A.tiles_m;
    if (nwg < 256) return launch_gemm_a8k_16(w, a, rows, total_rows, x, bias, y, stream);
    if (nwg > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nwg), block(512);
    if (w.dt == DT_Q4_K) hipLaunchKernelGGL((gemm_a8k_kernel<DT_Q4_K, 4, 2>), grid, block, 0, stream, A);
    else hipLaunchKernelGGL((gemm_a8k_kernel<DT_Q6_K, 4, 2>), grid, block, 0, stream, A);
    return hipGetLastError();
}

}  // namespace mimg
