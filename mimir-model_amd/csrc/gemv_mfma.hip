// Decode GEMV for 4..8 activation rows (dequant_matmul_a8.v2, block = 256;
// correct for 2..8) on the int8 matrix cores. At these row counts the pair
// kernel's integer dot products (eight lanes per (row, block, activation
// row)) cost more VALU time than the weights take to stream; one
// v_mfma_i32_16x16x64_i8 instead computes 16 weight rows x 16 activation
// rows x 64 k.
//
// Numerics: the same exact int32 block sums as the pair kernel and the GEMM
// (reference internal/kernels/q8k.go dotQ8KRef, q8k_test.go:38-102; the
// GEMM's split of the scaled weights into two int8 planes, gemm_kquant.hip),
// then per (weight row, activation row) the serial chain
// tot = fma(f32(S_b), d_b*dx_b, tot) (and off for Q4_K's mins) in block
// order: bit for bit the one-row kernel.
//
// Work split: a 256-thread workgroup owns 16 weight rows of one matrix. Its
// four waves take blocks w, w+4, w+8, ... (measured against two, eight and
// sixteen waves: four is fastest); per block a wave loads its A
// operand straight from the weights in their file layout (lane l: row l%16,
// the 16 k of group l/16 in each 64-k step), the B operand from the
// quantized activations (lane l: activation row l%16, rows past M clamped,
// their columns never read), runs 12 (Q4_K) or 8 (Q6_K) MFMAs and writes
// the block's exact (S, M) per (row, activation row) to an LDS table (Q6_K:
// with the next block's loads in flight). Then one lane per (row,
// activation row) runs the float chain over the table in block order.
// Rows of x the quantizer refused and weight rows with a non-finite block
// scale take the float32 path (reference interp/fast.go:323-377).
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int MF_ROWS = 16;  // weight rows per workgroup (the MFMA's A rows)
#ifndef MIMG_MF_WAVES
#define MIMG_MF_WAVES 4
#endif
constexpr int MF_WAVES = MIMG_MF_WAVES;  // waves per workgroup; they split the blocks
constexpr int MF_T = 64 * MF_WAVES;

struct MfmaMat {
    const uint8_t* W;
    const uint8_t* wref;  // [N]
    const float* bias;    // [N] or null
    float* y;             // [M][N]
    int N;
    int tile0;            // first workgroup of this matrix
};

struct MfmaArgs {
    MfmaMat mat[3];
    int nmat;
    int64_t rb;          // bytes per weight row
    int nb, M;           // blocks per row, activation rows (2..8)
    int64_t K;
    const int8_t* q;     // [M][K]
    const float* d32;    // [M][K/32]
    const int32_t* ok;   // [M]
    const float* x;      // [M][K] f32 (float32 path)
    int fused;           // float32 path order: total rows <= 8
};

// One lane's loads for one block (all unconditional, in bounds).
template <uint32_t DT>
struct MfRaw;
template <>
struct MfRaw<DT_Q4_K> {
    u32x4 hdr;     // d, dmin, the 12 scale bytes of row l%16
    u32x4 qs[4];   // per 64-k step: the 16 bytes whose nibbles are this lane's k
    v4i act[4];    // per 64-k step: 16 int8 activations
    float dx;      // the block's activation scale (row l%16)
};
template <>
struct MfRaw<DT_Q6_K> {
    uint32_t ql[2][5], qh[2][5];  // per half: 16 bytes as the 5 aligned dwords holding them
    int sc[4];                    // per 64-k step: the sub-block scale
    uint32_t dbits, shift;
    v4i act[4];
    float dx;
};

template <uint32_t DT>
__device__ __forceinline__ void mf_load(const uint8_t* Wt, uint32_t roff, int b, const int8_t* ya,
                                        const float* dxr, int G, MfRaw<DT>& r) {
    if constexpr (DT == DT_Q4_K) {
        const uint32_t off = roff + (uint32_t)b * Q4K_BYTES;  // 16-byte aligned
        r.hdr = *(const u32x4*)(Wt + off);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) r.qs[ks] = *(const u32x4*)(Wt + (off + 16 + 32 * ks + 16 * (G & 1)));
    } else {
        const uint32_t off = roff + (uint32_t)b * Q6K_BYTES;  // 2-byte aligned
        r.shift = off & 3;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t oa = (off + 64 * h + 16 * G) & ~3u;
            const uint32_t oc = (off + 128 + 32 * h + 16 * (G & 1)) & ~3u;
            const u32x4a4 av = *(const u32x4a4*)(Wt + oa), cv = *(const u32x4a4*)(Wt + oc);
            r.ql[h][0] = av.x, r.ql[h][1] = av.y, r.ql[h][2] = av.z, r.ql[h][3] = av.w;
            r.ql[h][4] = *(const uint32_t*)(Wt + oa + 16);
            r.qh[h][0] = cv.x, r.qh[h][1] = cv.y, r.qh[h][2] = cv.z, r.qh[h][3] = cv.w;
            r.qh[h][4] = *(const uint32_t*)(Wt + oc + 16);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int h = ks >> 1, p = 2 * (ks & 1) + (G >> 1);
            r.sc[ks] = (int)*(const int8_t*)(Wt + (off + 192 + 8 * h + (G & 1) + 2 * p));
        }
        r.dbits = *(const uint16_t*)(Wt + (off + 208));
    }
    const int8_t* yb = ya + (uint32_t)b * 256;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) r.act[ks] = *(const v4i*)(yb + 64 * ks + 16 * G);
    r.dx = dxr[8 * b];
}

// The block's exact sums: lane l holds, for weight rows 4(l/16) + i (i <
// 4) and activation row l%16, S in s[i] and (Q4_K) the mins term in mt[i].
template <uint32_t DT>
__device__ __forceinline__ void mf_block(const MfRaw<DT>& r, int G, v4i& s, v4i& mt) {
    v4i accH = {0, 0, 0, 0}, accL = {0, 0, 0, 0}, accM = {0, 0, 0, 0};
    if constexpr (DT == DT_Q4_K) {
        const Q4KScales S = q4k_scales(r.hdr.y, r.hdr.z, r.hdr.w);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            // sub-block 2ks (low nibbles, G < 2) or 2ks+1 (high nibbles); its
            // scale sc = 8*sh + sl with sh, sl <= 7, so sh*q and sl*q (q <= 15)
            // are bytes: the packed nibbles times a small constant in 16-bit lanes
            const int sub = 2 * ks + (G >> 1);
            const uint32_t sc = byte_of(S.sc, sub), mm = byte_of(S.m, sub);
            const short sh = (short)(sc >> 3), sl = (short)(sc & 7);
            const s16x2 shp = {sh, sh}, slp = {sl, sl};
            const int shift = 4 * (G >> 1);
            const uint32_t qd[4] = {r.qs[ks].x, r.qs[ks].y, r.qs[ks].z, r.qs[ks].w};
            v4i aH, aL, aM;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const s16x2 nib = as_s16x2((qd[k] >> shift) & 0x0F0F0F0Fu);
                aH[k] = (int)as_u32(nib * shp);
                aL[k] = (int)as_u32(nib * slp);
                aM[k] = (int)(mm * 0x01010101u);
            }
            accH = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, r.act[ks], accH, 0, 0, 0);
            accL = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, r.act[ks], accL, 0, 0, 0);
            accM = __builtin_amdgcn_mfma_i32_16x16x64_i8(aM, r.act[ks], accM, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = (accH[i] << 3) + accL[i];
        mt = accM;
    } else {
        uint32_t ql[2][4], qh[2][4];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                ql[h][k] = __builtin_amdgcn_alignbyte(r.ql[h][k + 1], r.ql[h][k], r.shift);
                qh[h][k] = __builtin_amdgcn_alignbyte(r.qh[h][k + 1], r.qh[h][k], r.shift);
            }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            // w = sc*(q - 32) in [-4096, 4064] as 128*hi + lo, lo in [0, 127]
            const int h = ks >> 1, p = 2 * (ks & 1) + (G >> 1);
            const s16x2 sc2 = {(short)r.sc[ks], (short)r.sc[ks]};
            v4i aH, aL;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t q6 = (((ks & 1) ? (ql[h][k] >> 4) : ql[h][k]) & 0x0F0F0F0Fu) |
                                    (((qh[h][k] >> (2 * p)) & 0x03030303u) << 4);
                const s16x2 we = (as_s16x2(q6 & 0x00FF00FFu) - (s16x2){32, 32}) * sc2;
                const s16x2 wo = (as_s16x2((q6 >> 8) & 0x00FF00FFu) - (s16x2){32, 32}) * sc2;
                uint32_t lo, hi;
                split4(as_u32(we), as_u32(wo), as_u32(we >> (s16x2){7, 7}), as_u32(wo >> (s16x2){7, 7}), lo, hi);
                aL[k] = (int)lo;
                aH[k] = (int)hi;
            }
            accH = __builtin_amdgcn_mfma_i32_16x16x64_i8(aH, r.act[ks], accH, 0, 0, 0);
            accL = __builtin_amdgcn_mfma_i32_16x16x64_i8(aL, r.act[ks], accL, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = (accH[i] << 7) + accL[i];
        mt = accM;
    }
}

// LDS: the (S, M) table [nb][16][M] (int2; Q6_K int), the block scales'
// f16 bits per (block, row), dx per (block, activation row) and the
// refusal flag per (row, activation row).
template <uint32_t DT>
__host__ __device__ constexpr size_t mf_lds_bytes(int nb, int M) {
    return (size_t)nb * MF_ROWS * M * (DT == DT_Q4_K ? 8 : 4) + (size_t)nb * MF_ROWS * 4 + (size_t)nb * M * 4 +
           (size_t)MF_ROWS * M * 4;
}

template <uint32_t DT>
__global__ __launch_bounds__(MF_T) void gemv_a8k_mfma_kernel(MfmaArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    int mi = 0;
    if (A.nmat > 1 && (int)blockIdx.x >= A.mat[1].tile0) mi = 1;
    if (A.nmat > 2 && (int)blockIdx.x >= A.mat[2].tile0) mi = 2;
    const MfmaMat P = mi == 0 ? A.mat[0] : mi == 1 ? A.mat[1] : A.mat[2];
    const int t = threadIdx.x, l = t & 63, ar = l & 15, G = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the block loop is scalar
    const int nb = A.nb, M = A.M, N = P.N;
    const int row0 = ((int)blockIdx.x - P.tile0) * MF_ROWS;
    constexpr int TW = DT == DT_Q4_K ? 2 : 1;  // table words per entry
    int* tab = (int*)smem;                                        // [nb][16][M][TW]
    uint32_t* dd = (uint32_t*)(tab + (size_t)nb * MF_ROWS * M * TW);  // [nb][16]
    float* dxs = (float*)(dd + (size_t)nb * MF_ROWS);                 // [nb][M]
    int* refl = (int*)(dxs + (size_t)nb * M);                         // [16][M]

    // The tile's rows from a 4-byte-aligned base (Q6_K rows may be 2-byte
    // aligned) with 32-bit offsets; rows past N read the last row.
    const int64_t tbyte = (int64_t)row0 * A.rb;
    const uint8_t* Wt = P.W + (tbyte & ~(int64_t)3);
    const uint32_t roff = (uint32_t)(tbyte & 3) + (uint32_t)min(ar, N - 1 - row0) * (uint32_t)A.rb;
    const int am = min(ar, M - 1);
    const int8_t* ya = A.q + (int64_t)am * A.K;
    const float* dxr = A.d32 + (int64_t)am * (A.K / 32);

    // Lane t < 16*M owns (row t/M, activation row t%M) at the end. Its
    // flags and bias are loaded first and looked at last (loaded after the
    // weights, they would wait for all of them).
    const int ft = min(t, MF_ROWS * M - 1), fr = ft / M;
    int fm = ft - fr * M;
    asm volatile("v_mov_b32 %0, %1" : "=v"(fm) : "v"(fm));  // a vector index: ok[] through the vector cache
    const int frow = min(row0 + fr, N - 1);
    const int wr = P.wref[frow], okm = A.ok[fm];
    const float bias = P.bias ? P.bias[frow] : 0.f;
    __builtin_amdgcn_sched_barrier(0);

    // Block b's table entries, scale bits and dx.
    auto step = [&](const MfRaw<DT>& r, int b) {
        v4i s, mt;
        mf_block<DT>(r, G, s, mt);
        if (ar < M) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int* e = tab + (((size_t)b * MF_ROWS + 4 * G + i) * M + ar) * TW;
                e[0] = s[i];
                if constexpr (DT == DT_Q4_K) e[1] = mt[i];
            }
        }
        if (G == 0) {
            if constexpr (DT == DT_Q4_K) dd[b * MF_ROWS + ar] = r.hdr.x;
            else dd[b * MF_ROWS + ar] = r.dbits;
        }
        if (G == 1 && ar < M) dxs[b * M + ar] = r.dx;
    };
    // Everything block b needs is loaded with it (the load counter retires
    // in order: a load issued after the next block's would make this block
    // wait for all of them), and sched_barrier keeps the scheduler from
    // sinking the next block's loads below this block's arithmetic.
    if constexpr (DT == DT_Q4_K) {
        // One block in flight per wave: 88 registers against 128, so more
        // waves (measured: 19.1 against 21.7 us for gate at 8 rows).
        for (int b = w; b < nb; b += MF_WAVES) {
            MfRaw<DT> r1;
            mf_load<DT>(Wt, roff, b, ya, dxr, G, r1);
            __builtin_amdgcn_sched_barrier(0);
            step(r1, b);
        }
    } else {
        // Q6_K (seven loads per 16 bytes of weights): two sets of registers
        // in turn, block b computing while block b + MF_WAVES loads (a copy
        // from one set to the other would wait for its loads); measured
        // 24.3 against 26.2 us for down at 8 rows.
        MfRaw<DT> ra, rb;
        mf_load<DT>(Wt, roff, min(w, nb - 1), ya, dxr, G, ra);
        for (int b = w; b < nb; b += 2 * MF_WAVES) {
            mf_load<DT>(Wt, roff, min(b + MF_WAVES, nb - 1), ya, dxr, G, rb);
            __builtin_amdgcn_sched_barrier(0);
            step(ra, b);
            if (b + MF_WAVES >= nb) break;  // uniform within the wave
            mf_load<DT>(Wt, roff, min(b + 2 * MF_WAVES, nb - 1), ya, dxr, G, ra);
            __builtin_amdgcn_sched_barrier(0);
            step(rb, b + MF_WAVES);
        }
    }
    const int flag = (wr != 0) | (okm == 0);
    if (t < MF_ROWS * M) refl[t] = flag;
    __syncthreads();

    // The serial float chain, one lane per (weight row, activation row).
    if (t < MF_ROWS * M) {
        const int r = t / M, m = t - r * M, row = row0 + r;
        if (row < N && !flag) {
            float tot = 0.f, off = 0.f;
            for (int b = 0; b < nb; b++) {
                const int* e = tab + (((size_t)b * MF_ROWS + r) * M + m) * TW;
                const uint32_t bits = dd[b * MF_ROWS + r];
                const float dx = dxs[b * M + m];
                tot = __builtin_fmaf((float)e[0], f16_to_f32(bits & 0xFFFFu) * dx, tot);
                if constexpr (DT == DT_Q4_K) off = __builtin_fmaf((float)e[1], f16_to_f32(bits >> 16) * dx, off);
            }
            float res = DT == DT_Q4_K ? tot - off : tot;
            if (P.bias) res += bias;
            P.y[(int64_t)m * N + row] = res;
        }
    }
    // The float32 path for refused pairs, one group of eight lanes per pair.
    const int g = t >> 3;
    for (int qq = g; qq < MF_ROWS * M; qq += MF_T / 8) {
        const int r = qq / M, m = qq - r * M, row = row0 + r;
        if (row < N && refl[qq]) {
            float res = f32dot_g8<DT>(P.W + (int64_t)row * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
            if (P.bias) res += P.bias[row];
            if ((t & 7) == 0) P.y[(int64_t)m * N + row] = res;
        }
    }
}

bool gemv_mfma_ok(const DevWeight* const* ws, int nmat, int64_t rows) {
    if (rows < 2 || rows > 8 || nmat < 1 || nmat > 3) return false;
    const DevWeight& w = *ws[0];
    if ((w.dt != DT_Q4_K && w.dt != DT_Q6_K) || w.k % 256 || w.k <= 0) return false;
    for (int i = 0; i < nmat; i++)
        if (ws[i]->dt != w.dt || ws[i]->k != w.k || ws[i]->n <= 0) return false;
    const int nb = (int)(w.k / 256);
    const size_t lds = w.dt == DT_Q4_K ? mf_lds_bytes<DT_Q4_K>(nb, (int)rows) : mf_lds_bytes<DT_Q6_K>(nb, (int)rows);
    return lds <= 64 * 1024;
}

hipError_t launch_gemv_a8k_mfma(const DevWeight* const* ws, int nmat, const ActPtrs& a, int64_t rows,
                                int64_t total_rows, const float* x, const float* const* bias, float* const* y,
                                hipStream_t stream) {
    if (!gemv_mfma_ok(ws, nmat, rows)) return hipErrorInvalidValue;
    const DevWeight& w = *ws[0];
    MfmaArgs A;
    A.nmat = nmat;
    A.rb = w.row_bytes;
    A.nb = (int)(w.k / 256);
    A.M = (int)rows;
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    int tiles = 0;
    for (int i = 0; i < 3; i++) {
        const DevWeight& wi = *ws[i < nmat ? i : 0];
        A.mat[i].W = wi.data;
        A.mat[i].wref = wi.wref;
        A.mat[i].bias = i < nmat ? bias[i] : nullptr;
        A.mat[i].y = i < nmat ? y[i] : nullptr;
        A.mat[i].N = (int)wi.n;
        A.mat[i].tile0 = tiles;
        if (i < nmat) tiles += (int)((wi.n + MF_ROWS - 1) / MF_ROWS);
    }
    if (w.dt == DT_Q4_K)
        hipLaunchKernelGGL(gemv_a8k_mfma_kernel<DT_Q4_K>, dim3((unsigned)tiles), dim3(MF_T),
                           mf_lds_bytes<DT_Q4_K>(A.nb, A.M), stream, A);
    else
        hipLaunchKernelGGL(gemv_a8k_mfma_kernel<DT_Q6_K>, dim3((unsigned)tiles), dim3(MF_T),
                           mf_lds_bytes<DT_Q6_K>(A.nb, A.M), stream, A);
    return hipGetLastError();
}

}  // namespace mimg
