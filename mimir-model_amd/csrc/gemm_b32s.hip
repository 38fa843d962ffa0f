// The opt-in activation-blocks-of-32 GEMMs (Q8_0: gemm_q8_0.hip; Q4_K /
// Q6_K: gemm_kq_b32.hip) for small grids: 16 weight rows x 64 activation
// rows per workgroup of four waves on v_mfma_i32_16x16x32_i8, so that a
// grid of few weight rows (down: 4096) or few activation rows still has a
// workgroup for every CU and four waves in each. The per-output arithmetic
// is the other tilings' exactly (same exact int32 block sums, same float
// steps in the same order), so a row's result does not depend on the tiling
// the call's shape selects:
//   Q8_0  tot = fma(f32(S_j), f32(d_j) * dx_j, tot) over the blocks j in order;
//   Q4_K  per weight block: t = fma(f32(sc_j * P_j), dx_j, t) over its 8
//         activation blocks, tot = fma(d, t, tot); off = fma(dmin * f32(m_j),
//         dbs_j, off) per j; result tot - off;
//   Q6_K  as Q4_K with S_j = sc_2j * P_2j + sc_2j+1 * P_2j+1 over the two
//         sub-blocks of 16, no off;
// plus the bias; refused rows take the reference's float32 path.
//
// Operands: the activations are the MFMA's A operand (lane l: activation row
// l % 16 of the wave's 16, the 8 k of group l / 16) and the weights the B
// operand (column l % 16 = the lane's weight row), so a lane of the 16 x 16
// result holds activation rows 4(l/16) + i of its own weight row: one block
// scale per lane and block, the activation scales as one float4. Per group
// of 8 activation blocks (256 elements) the weight rows' bytes, the int8
// activation rows (16-byte chunks XOR-swizzled by row) and the rows' dx (and
// dbs) are copied into LDS with global_load_lds, a ring of NS stages; all
// four waves read the same weights.
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {
namespace b32s {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef long v1l;

constexpr int T = 256, BN = 16, BM = 64;

// AL: every weight group starts at a 16-byte boundary (Q4_K always; Q8_0
// when the data pointer is 16-byte aligned: a row of K elements is
// 272 K / 256 bytes), so the blocks' offsets within a slot are constants.
template <uint32_t DT, bool AL>
struct Lay {
    static constexpr int GB = DT == DT_Q8_0 ? 8 * Q80_BYTES : DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    // 16-byte chunks of a weight row's slot per group of 256 elements: Q8_0
    // 8 blocks of 34 bytes (aligned: 17 chunks; 2-byte aligned: 18 chunks
    // from the 16-byte boundary below cover them), Q4_K one block (9
    // chunks), Q6_K one block (14 chunks from the boundary below); the
    // unaligned Q8_0 and Q6_K slots take one chunk more (copied too), an odd
    // count, so that the 16 rows' dword reads spread over the banks.
    static constexpr int WCH = DT == DT_Q8_0 ? (AL ? 17 : 19) : DT == DT_Q4_K ? 9 : 15;
    static constexpr int WSLOT = 16 * WCH;
    static constexpr int WDMA = (BN * WCH + T - 1) / T;
    static constexpr int WBYTES = WDMA * T * 16;
    static constexpr int ADMA = BM * 16 / T;
    static constexpr int ABYTES = BM * 256;
    static constexpr int XDMA = BM * 8 / T;
    static constexpr int XBYTES = BM * 8 * 4;
    static constexpr int YDMA = DT == DT_Q4_K ? XDMA : 0;
    static constexpr int YBYTES = DT == DT_Q4_K ? XBYTES : 0;
    static constexpr int BUF = WBYTES + ABYTES + XBYTES + YBYTES;
    static constexpr int NDMA = WDMA + ADMA + XDMA + YDMA;
    static_assert(ADMA * T == BM * 16 && XDMA * T == BM * 8, "small block-32 tile");
    static constexpr int NS = 2;  // stages of the copy ring (NS - 1 groups in flight; 3 and 4 measured slower)
    static_assert(NS * BUF <= 160 * 1024 && (NS - 1) * NDMA < 64, "small block-32 buffers");
};

struct Args {
    const uint8_t* W;
    const uint8_t* wref;
    const float* bias;
    float* y;
    int64_t rb;
    int N, M, ng;          // groups of 256 elements per row
    int64_t K;
    const int8_t* q;
    const float* d32;
    const float* dbs;
    const int32_t* ok;
    const float* x;
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
#define BS_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define BS_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)
__device__ __forceinline__ void bs_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A thread's copy sources for group 0, fixed over the groups (group gi adds
// gi times a row's group stride).
template <uint32_t DT, bool AL>
struct CopySrc {
    const uint8_t* w[Lay<DT, AL>::WDMA];  // its weight chunk (AL), else its row's group 0
    int wch[Lay<DT, AL>::WDMA];           // the chunk within the slot (not AL)
    const int8_t* a[Lay<DT, AL>::ADMA];   // its activation chunk
    const float* x[Lay<DT, AL>::XDMA];    // its dx (and dbs at the same index)
};

template <uint32_t DT, bool AL>
__device__ __forceinline__ CopySrc<DT, AL> copy_sources(const Args& A, int n0, int m0) {
    using L = Lay<DT, AL>;
    const int t = threadIdx.x;
    CopySrc<DT, AL> cs;
#pragma unroll
    for (int i = 0; i < L::WDMA; i++) {
        const int c = min(T * i + t, BN * L::WCH - 1);
        const int r = c / L::WCH, j = c - L::WCH * r;
        cs.w[i] = A.W + (int64_t)min(n0 + r, A.N - 1) * A.rb + (AL ? 16 * j : 0);
        cs.wch[i] = j;
    }
#pragma unroll
    for (int i = 0; i < L::ADMA; i++) {
        const int c = T * i + t;  // row c/16, chunk c%16 stored at slot (c%16) ^ (row & 15)
        const int r = c >> 4, s = c & 15;
        cs.a[i] = A.q + (int64_t)min(m0 + r, A.M - 1) * A.K + 16 * (s ^ (r & 15));
    }
#pragma unroll
    for (int i = 0; i < L::XDMA; i++) {
        const int c = T * i + t;  // block j = c / BM, activation row c % BM
        const int j = c / BM, r = c - BM * j;
        cs.x[i] = A.d32 + (int64_t)min(m0 + r, A.M - 1) * (A.K / 32) + j;
    }
    return cs;
}

template <uint32_t DT, bool AL>
__device__ __forceinline__ void issue_group(const Args& A, const CopySrc<DT, AL>& cs, int gi, uint8_t* buf) {
    using L = Lay<DT, AL>;
    const int wave = threadIdx.x >> 6;
    uint8_t* wl = buf;
    uint8_t* al = buf + L::WBYTES;
    uint8_t* xl = al + L::ABYTES;
#pragma unroll
    for (int i = 0; i < L::WDMA; i++) {
        const uint8_t* g = cs.w[i] + (int64_t)L::GB * gi;
        const uint8_t* src = AL ? g : (const uint8_t*)__builtin_align_down(g, 16) + 16 * cs.wch[i];
        lds_copy16(src, wl + 16 * (T * i + 64 * wave));
    }
#pragma unroll
    for (int i = 0; i < L::ADMA; i++) lds_copy16(cs.a[i] + 256 * (int64_t)gi, al + 16 * (T * i + 64 * wave));
#pragma unroll
    for (int i = 0; i < L::XDMA; i++) {
        lds_copy4(cs.x[i] + 8 * gi, xl + 4 * (T * i + 64 * wave));
        if constexpr (DT == DT_Q4_K)
            lds_copy4(A.dbs + (cs.x[i] - A.d32) + 8 * gi, xl + L::XBYTES + 4 * (T * i + 64 * wave));
    }
}

// 8 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ v1l lds_read8_a2(const uint8_t* p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, sh), hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return (v1l)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ uint32_t lds_u16_a2(const uint8_t* p) {
    const uint32_t* w = (const uint32_t*)__builtin_align_down(p, 4);
    return (w[0] >> (8 * ((uint32_t)(uintptr_t)p & 2))) & 0xFFFFu;
}

// Q8_0 block j of a group that starts 16-byte aligned: its bytes 8G..8G+7
// (B operand) and its scale, with the offsets mod 4 known (block j at 34 j;
// j is a constant once the block loop is unrolled).
__device__ __forceinline__ void q80_block_al(const uint8_t* wr, int j, int G, v1l& bw, float& dj) {
    const uint8_t* blk = wr + Q80_BYTES * j;
    if (j & 1) {
        const uint32_t* p = (const uint32_t*)(blk + 2 + 8 * G);  // 34 j + 2: a multiple of 4
        bw = (v1l)(((uint64_t)p[1] << 32) | p[0]);
        dj = f16_to_f32(((const uint32_t*)(blk - 2))[0] >> 16);
    } else {
        const uint32_t* p = (const uint32_t*)(blk + 8 * G);  // 34 j: a multiple of 4
        const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
        bw = (v1l)(((uint64_t)__builtin_amdgcn_alignbyte(w2, w1, 2) << 32) | __builtin_amdgcn_alignbyte(w1, w0, 2));
        dj = f16_to_f32(((const uint32_t*)blk)[0]);
    }
}

template <uint32_t DT, bool AL>
__global__ __launch_bounds__(T) void b32s_kernel(Args A) {
    using L = Lay<DT, AL>;
    constexpr int NS = L::NS;
    __shared__ __align__(16) uint8_t smem[NS * L::BUF];
    __shared__ int flags[1];
    const int t = threadIdx.x, l = t & 63, wave = t >> 6;
    const int ar = l & 15, G = l >> 4;
    const int ntn = (A.N + BN - 1) / BN;
    const int nwg = ntn * A.tiles_m;
    int wg = blockIdx.x;
    if (nwg % 8 == 0) wg = (wg % 8) * (nwg / 8) + wg / 8;  // the row tiles of a weight tile on one XCD
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
    // This lane's weight row (its B column) and the offset of its groups in
    // their slots (the copies start at the 16-byte boundary below a group).
    const uint32_t goff0 = (uint32_t)(uintptr_t)(A.W + (int64_t)min(n0 + ar, A.N - 1) * A.rb) & 15u;
    constexpr uint32_t GB = L::GB;
    const int arow = 16 * wave + ar;  // this lane's activation row of the tile (A operand)
    const CopySrc<DT, AL> cs = copy_sources<DT, AL>(A, n0, m0);
    float tot[4] = {0.f, 0.f, 0.f, 0.f}, off[4] = {0.f, 0.f, 0.f, 0.f};

    // The ring: groups 0 .. NS-2 first; at group gi, group gi + NS - 1 goes
    // into the stage group gi - 1 used (every wave is past it: the barrier
    // that ends group gi - 1). Past the last group the last one is copied
    // again, so every thread always has the same number of copies in flight.
#pragma unroll
    for (int i = 0; i < NS - 1; i++) issue_group<DT, AL>(A, cs, min(i, A.ng - 1), smem + i * L::BUF);
    for (int gi = 0; gi < A.ng; gi++) {
        uint8_t* buf = smem + (gi % NS) * L::BUF;
        issue_group<DT, AL>(A, cs, min(gi + NS - 1, A.ng - 1), smem + ((gi + NS - 1) % NS) * L::BUF);
        BS_WAIT_VMCNT((NS - 1) * L::NDMA);  // group gi's copies (issued NS - 1 groups earlier) have landed
        bs_barrier();
        const uint8_t* al = buf + L::WBYTES;
        const float* xl = (const float*)(al + L::ABYTES);
        const float* yl = xl + BM * 8;
        const uint8_t* wg0 = buf + ar * L::WSLOT + (AL ? 0u : ((goff0 + (uint32_t)gi * GB) & 15u));  // the lane's group
        float tb[4] = {0.f, 0.f, 0.f, 0.f};
        float d = 0.f, dmin = 0.f;
        Q4KScales sq = {0, 0};
        if constexpr (DT == DT_Q4_K) {
            const uint32_t* w4 = (const uint32_t*)wg0;  // 16-byte aligned block
            d = f16_to_f32(w4[0] & 0xFFFFu);
            dmin = f16_to_f32(w4[0] >> 16);
            sq = q4k_scales(w4[1], w4[2], w4[3]);
        } else if constexpr (DT == DT_Q6_K) {
            d = f16_to_f32(lds_u16_a2(wg0 + 208));
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            // A: activation row arow, k 32j + 8G .. + 7
            const v1l av = *(const v1l*)(al + arow * 256 + 16 * ((2 * j + (G >> 1)) ^ (arow & 15)) + 8 * (G & 1));
            const float4 dx4 = *(const float4*)(xl + BM * j + 16 * wave + 4 * G);
            const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const v4i z = {0, 0, 0, 0};
            if constexpr (DT == DT_Q8_0) {
                v1l bw;
                float dj;
                if constexpr (AL) {
                    q80_block_al(wg0, j, G, bw, dj);
                } else {
                    const uint8_t* blk = wg0 + Q80_BYTES * j;
                    bw = lds_read8_a2(blk + 2 + 8 * G);
                    dj = f16_to_f32(lds_u16_a2(blk));
                }
                const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bw, z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) tot[i] = __builtin_fmaf((float)c[i], dj * dxr[i], tot[i]);
            } else if constexpr (DT == DT_Q4_K) {
                const uint2 raw = *(const uint2*)(wg0 + 16 + 32 * (j >> 1) + 8 * G);
                const uint32_t sh = 4 * (j & 1);
                const v1l bw = (v1l)(((uint64_t)((raw.y >> sh) & 0x0F0F0F0Fu) << 32) | ((raw.x >> sh) & 0x0F0F0F0Fu));
                const int sc = (int)byte_of(sq.sc, j);
                const float dm = dmin * (float)byte_of(sq.m, j);
                const float4 db4 = *(const float4*)(yl + BM * j + 16 * wave + 4 * G);
                const float dbr[4] = {db4.x, db4.y, db4.z, db4.w};
                const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bw, z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    tb[i] = __builtin_fmaf((float)__mul24(sc, c[i]), dxr[i], tb[i]);
                    off[i] = __builtin_fmaf(dm, dbr[i], off[i]);
                }
            } else {
                // Q6_K: activation block j = half hn, run seg of 32; lanes
                // G < 2 hold sub-block 2j (k < 16), G >= 2 sub-block 2j+1
                const int hn = j >> 2, seg = j & 3;
                const v1l ql = lds_read8_a2(wg0 + 64 * hn + 32 * (seg & 1) + 8 * G);
                const v1l qh = lds_read8_a2(wg0 + 128 + 32 * hn + 8 * G);
                const uint64_t v = (((uint64_t)ql >> (4 * (seg >> 1))) & 0x0F0F0F0F0F0F0F0Full) |
                                   ((((uint64_t)qh >> (2 * seg)) & 0x0303030303030303ull) << 4);
                // q - 32 in each byte (q <= 63): set the top bit, subtract 32
                // (no borrow between bytes), flip the top bit back
                const uint64_t w = ((v | 0x8080808080808080ull) - 0x2020202020202020ull) ^ 0x8080808080808080ull;
                const v1l w0 = G < 2 ? (v1l)w : (v1l)0, w1 = G < 2 ? (v1l)0 : (v1l)w;
                const uint32_t sw = lds_u16_a2(wg0 + 192 + 8 * hn + 2 * seg);
                const int sa = (int)(int8_t)(sw & 0xFFu), sb = (int)(int8_t)(sw >> 8);
                const v4i ca = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, w0, z, 0, 0, 0);
                const v4i cb = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, w1, z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    tb[i] = __builtin_fmaf((float)(__mul24(sa, ca[i]) + __mul24(sb, cb[i])), dxr[i], tb[i]);
            }
        }
        if constexpr (DT != DT_Q8_0) {
#pragma unroll
            for (int i = 0; i < 4; i++) tot[i] = __builtin_fmaf(d, tb[i], tot[i]);
        }
        BS_WAIT_LGKM0();
        bs_barrier();  // stage gi % NS is reloaded in the next iteration
    }
    BS_WAIT_VMCNT(0);  // the ring's extra copies have landed before the workgroup's LDS is given back

    const int n = n0 + ar;
    const int refused = flags[0];
    if (n < A.N && !(refused && A.wref[n] != 0)) {
        const float bn = A.bias ? A.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + 16 * wave + 4 * G + i;
            if (m >= A.M) continue;
            if (refused && A.ok[m] == 0) continue;
            float res = DT == DT_Q4_K ? tot[i] - off[i] : tot[i];
            if (A.bias) res += bn;
            A.y[(int64_t)m * A.N + n] = res;
        }
    }
    if (!refused) return;
    // Refused pairs of the tile: the reference's float32 path.
    const int grp = t >> 3;
    for (int pidx = grp; pidx < BN * BM; pidx += T / 8) {
        const int nn = n0 + pidx % BN, m = m0 + pidx / BN;
        if (nn >= A.N || m >= A.M) continue;
        if (A.wref[nn] == 0 && A.ok[m] != 0) continue;
        float res = f32dot_g8<DT>(A.W + (int64_t)nn * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
        if (A.bias) res += A.bias[nn];
        if ((t & 7) == 0) A.y[(int64_t)m * A.N + nn] = res;
    }
}

}  // namespace b32s

// Workgroups the small tiling gives a product.
int64_t gemm_b32_small_wgs(int64_t n, int64_t rows) {
    return (n + b32s::BN - 1) / b32s::BN * ((rows + b32s::BM - 1) / b32s::BM);
}

hipError_t launch_gemm_b32_small(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows,
                                 const float* x, const float* bias, float* y, hipStream_t stream) {
    using namespace b32s;
    if ((w.dt != DT_Q8_0 && w.dt != DT_Q4_K && w.dt != DT_Q6_K) || w.k % 256 || w.k <= 0 || rows <= 0 ||
        rows > (1 << 30) || w.n > (1 << 30))
        return hipErrorInvalidValue;
    const bool al16 = ((uintptr_t)w.data & 15) == 0 && w.row_bytes % 16 == 0;
    if (w.dt == DT_Q4_K && !al16) return hipErrorInvalidValue;
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
    A.dbs = a.dbs;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    A.tiles_m = (int)((rows + BM - 1) / BM);
    const int64_t nwg = gemm_b32_small_wgs(w.n, rows);
    if (nwg > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nwg);
    if (w.dt == DT_Q8_0 && al16) hipLaunchKernelGGL((b32s_kernel<DT_Q8_0, true>), grid, dim3(T), 0, stream, A);
    else if (w.dt == DT_Q8_0) hipLaunchKernelGGL((b32s_kernel<DT_Q8_0, false>), grid, dim3(T), 0, stream, A);
    else if (w.dt == DT_Q4_K) hipLaunchKernelGGL((b32s_kernel<DT_Q4_K, true>), grid, dim3(T), 0, stream, A);
    else hipLaunchKernelGGL((b32s_kernel<DT_Q6_K, false>), grid, dim3(T), 0, stream, A);
    return hipGetLastError();
}

}  // namespace mimg
