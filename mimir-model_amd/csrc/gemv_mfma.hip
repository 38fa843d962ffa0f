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
// Work split: a workgroup owns 16 weight rows of one matrix; its NW waves
// (4; for Q6_K on small grids 8 or 12) take blocks w, w+NW, w+2NW, ...
// A wave's MFMA operand is 16 rows
// x 16 bytes per lane, and loads in that layout touch 16 rows 2-3 KB apart
// in every instruction (measured on MI355X: 31 us for the 66 MB of gate+up
// at 8 rows, against 17-18 us for the same bytes loaded 64 consecutive
// chunks per instruction, whether the runs are 144 bytes or whole rows).
// So a wave loads its block's 16 x 144 (Q4_K) or 16 x 224 (Q6_K, from the
// 16-byte boundary below each row's block) bytes as consecutive 16-byte
// chunks, one block ahead, writes them to its own LDS region (rows an odd
// number of chunks apart, so the 16 rows start in different banks) and
// reads its operand back in MFMA layout: no barrier, the wave's LDS
// accesses run in order. (A workgroup-wide staging of four blocks with a
// barrier per stage measured slower: 32 us without any arithmetic.) The
// activations (lane l: activation row l%16, rows past M clamped, their
// columns never read) come from global memory (L2-resident): straight into
// the B operand for Q4_K, through the wave's LDS region for Q6_K.
// Q4_K: per block 8 MFMAs with the activations as the A operand (each row
// of it one activation row's half of a 64-k step, so the 16 rows are 8
// activation rows x 2 sub-blocks) against the raw nibbles (the sub-block
// scales applied to the int32 results) and against the mins. Q6_K: the raw
// 6-bit values q (0..63) are the A operand, and
// the B operand puts each lane group's activation slice into its own four
// result columns, so one MFMA gives the per-16 sums of q*y for four
// sub-blocks apart; the sub-block scales are applied to those int32 sums
// (exact) and the -32 offset is one more MFMA with every A byte -32.
// A wave writes the block's
// exact (S, M) per (row, activation row) to an LDS table; then one lane per
// (row, activation row) runs the float chain over the table in block order.
// Rows of x the quantizer refused and weight rows with a non-finite block
// scale take the float32 path (reference interp/fast.go:323-377).
#include "decoder_math.hpp"
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int MF_ROWS = 16;  // weight rows per workgroup (the MFMA's A rows)

struct MfmaMat {
    const uint8_t* W;
    const uint8_t* wref;  // [N]
    const float* bias;    // [N] or null
    float* y;             // [M][N]
    int N;
    int tile0;            // first workgroup of this matrix
    int kind;             // MF_PLAIN, or the decoder epilogues below
};

// Epilogues of the attention input's products (rope.v1 and the cache
// scatter of rope_kv_kernel, with the head dim RD a template constant):
// q rotated to y, k rotated into the key cache, v into the value cache at
// the cache index of each activation row. The rows of q and k are dealt to
// workgroups in rotation pairs.
enum { MF_PLAIN = 0, MF_ROPE_Q = 1, MF_ROPE_K = 2, MF_STORE_V = 3 };

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
    // rope and cache scatter (matrices of another kind than MF_PLAIN)
    const int64_t* pos;   // [M]
    const int64_t* cidx;  // [M]
    const double* inv_freq;
    int rotary, interleaved, f16;
    int64_t C;
    void* kc;
    void* vc;
    // swiglu in the epilogue (mat[0] gate, mat[1] up): sw [M][N] = swiglu.v1
    // of the flattened [M][N] products with the reference's pieces
    float* sw;
    int64_t sw_total, sw_chunk;
};

// Row of local row r of tile `tile`: q and k rows in rotation pairs (local
// rows 2j, 2j+1 are dims (a, b) of pair P = 8 tile + j: head P / (RD/2),
// pair P % (RD/2), as rope_kv_kernel numbers them), other rows in order.
template <int RD>
__device__ __forceinline__ int mf_row(const MfmaArgs& A, const MfmaMat& P, int tile, int r) {
    if (RD == 0 || (P.kind != MF_ROPE_Q && P.kind != MF_ROPE_K)) return tile * 16 + r;
    constexpr int half = RD / 2;
    const int h2 = A.rotary / 2;
    const int Q = tile * 8 + (r >> 1), hh = Q / half, i = Q - hh * half;
    int a, b;
    if (A.interleaved) {
        a = 2 * i;
        b = a + 1;
    } else if (i < h2) {
        a = i;
        b = i + h2;
    } else {
        a = A.rotary + 2 * (i - h2);
        b = a + 1;
    }
    return hh * RD + ((r & 1) ? b : a);
}

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
    uint32_t dbits, shift;
};

// A wave's staging of one block: CPR 16-byte chunks per row (Q6_K blocks
// start 2-byte aligned: 14 chunks from the boundary below cover 210 bytes),
// stored RST chunks apart in the wave's LDS region.
// Q6_K also stages the block's activations: 8 rows AROW bytes apart (so
// the 16 lanes reading 4 rows x 4 k-slices of one B operand hit distinct
// banks), then 256 zero bytes for the lanes whose B operand is zero.
constexpr int Q6_AROW = 320;
template <uint32_t DT>
struct MfWave {
    static constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    static constexpr int CPR = DT == DT_Q4_K ? 9 : 14;
    static constexpr int RST = CPR | 1;
    static constexpr int CH = MF_ROWS * CPR;       // chunks per block
    static constexpr int NLD = (CH + 63) / 64;     // loads per lane and block
    static constexpr int WBYTES = MF_ROWS * RST * 16;
    static constexpr int LBYTES = WBYTES + (DT == DT_Q6_K ? 8 * Q6_AROW + 256 : 0);
};

// A lane's part of every block's loads: chunk q = 64i + lane (clamped to
// the last) of local row r = q / CPR (first byte rowptr(r)), stored at LDS
// byte 16 (RST r + j), j = q % CPR. Computed once per workgroup.
template <uint32_t DT>
struct MfLanes {
    const uint8_t* row[MfWave<DT>::NLD];  // the row's first byte (+16j for Q4_K)
    uint32_t j16[MfWave<DT>::NLD];        // 16j (Q6_K)
    uint32_t lds[MfWave<DT>::NLD];
    template <class RowPtr>
    __device__ MfLanes(RowPtr rowptr) {
        using S = MfWave<DT>;
        const int l = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < S::NLD; i++) {
            const int q = min(64 * i + l, S::CH - 1);
            const int r = q / S::CPR, j = q - S::CPR * r;
            row[i] = rowptr(r) + (DT == DT_Q4_K ? 16 * j : 0);
            j16[i] = 16 * j;
            lds[i] = 16 * (S::RST * r + j);
        }
    }
};

// Issues the loads of block b: Q4_K blocks are 16-byte aligned (rows and
// weight views are); Q6_K chunks count from the 16-byte boundary at or
// below the row's block and end at most 14 bytes past it (inside the next
// block, or WEIGHT_PAD past the matrix).
template <uint32_t DT>
__device__ __forceinline__ void mf_load_w(const MfLanes<DT>& L, int b, u32x4* v) {
    using S = MfWave<DT>;
#pragma unroll
    for (int i = 0; i < S::NLD; i++) {
        const uint8_t* p = L.row[i] + (int64_t)b * S::BYTES;
        if constexpr (DT == DT_Q6_K) p = (const uint8_t*)__builtin_align_down(p, 16) + L.j16[i];
        v[i] = *(const u32x4*)p;
    }
}

// Writes a block's chunks to the wave's LDS region (lanes past the last
// chunk write it again, the same bytes).
template <uint32_t DT>
__device__ __forceinline__ void mf_stage_w(const MfLanes<DT>& L, uint8_t* wl, const u32x4* v) {
#pragma unroll
    for (int i = 0; i < MfWave<DT>::NLD; i++) *(u32x4*)(wl + L.lds[i]) = v[i];
}

// A lane's weight operand for one block from the wave's LDS region; p is
// the block's first byte (Q4_K: 16-byte aligned; Q6_K: 2-byte aligned, read as
// aligned dwords and realigned in mf_block).
template <uint32_t DT>
__device__ __forceinline__ void mf_lds_w(const uint8_t* p, int G, MfRaw<DT>& r) {
    if constexpr (DT == DT_Q4_K) {
        r.hdr = *(const u32x4*)p;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) r.qs[ks] = *(const u32x4*)(p + 16 + 32 * ks + 16 * (G & 1));
    } else {
        r.shift = (uint32_t)(uintptr_t)p & 3;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t* qa = (const uint32_t*)__builtin_align_down(p + 64 * h + 16 * G, 4);
            const uint32_t* qc = (const uint32_t*)__builtin_align_down(p + 128 + 32 * h + 16 * (G & 1), 4);
#pragma unroll
            for (int k = 0; k < 5; k++) {
                r.ql[h][k] = qa[k];
                r.qh[h][k] = qc[k];
            }
        }
        r.dbits = *(const uint16_t*)(p + 208);
    }
}

// Q4_K, the block's exact sums. The activations are the A operand and the
// weights the B operand: A row a = l % 16 is activation row a/2's k-slice G
// when G/2 == a % 2 (the half of the 64-k step holding sub-block 2ks + a%2),
// zeros otherwise; B is the raw nibbles q of this lane's weight row l % 16.
// So C row a, column n is sum_{k in sub-block 2ks + a%2} q_k y_k of
// activation row a/2 and weight row n alone, and lane l (column l % 16 = its
// own weight row) holds rows 4G + i: the scale of its own row's sub-block
// 2ks + i%2 multiplies each (exact 24-bit products), and rows 2j, 2j+1 (the
// two halves) add up to activation row 2G + j. The mins term is a second
// MFMA with B = the sub-block's min m_s in every byte, accumulated over the
// k steps. Out: s[j], mt[j] for weight row l % 16, activation row 2G + j.
template <uint32_t DT>
__device__ __forceinline__ void mf_block(const MfRaw<DT>& r, int G, int ar, int (&s)[2], int (&mt)[2]) {
    if constexpr (DT == DT_Q4_K) {
        const Q4KScales S = q4k_scales(r.hdr.y, r.hdr.z, r.hdr.w);
        const v4i zero = {0, 0, 0, 0};
        const bool on = (G >> 1) == (ar & 1);  // this lane's A row carries its activation slice
        v4i accM = zero;
        int acc[4] = {0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int shift = 4 * (G >> 1);  // low nibbles for G < 2 (sub-block 2ks), high for G >= 2
            const uint32_t mm = byte_of(S.m, 2 * ks + (G >> 1));
            const uint32_t qd[4] = {r.qs[ks].x, r.qs[ks].y, r.qs[ks].z, r.qs[ks].w};
            v4i bq, bm;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                bq[k] = (int)((qd[k] >> shift) & 0x0F0F0F0Fu);
                bm[k] = (int)(mm * 0x01010101u);
            }
            const v4i av = on ? r.act[ks] : zero;
            const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq, zero, 0, 0, 0);
            accM = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bm, accM, 0, 0, 0);
            const int sc0 = (int)byte_of(S.sc, 2 * ks), sc1 = (int)byte_of(S.sc, 2 * ks + 1);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] += __mul24((i & 1) ? sc1 : sc0, c[i]);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            s[j] = acc[2 * j] + acc[2 * j + 1];
            mt[j] = accM[2 * j] + accM[2 * j + 1];
        }
    }
}

// Sum over the four lanes of a quad (exact: integers).
__device__ __forceinline__ int quad_sum(int x) {
    x += __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);  // quad_perm 1,0,3,2
    x += __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);  // quad_perm 2,3,0,1
    return x;
}

// Q6_K, the block's exact sums S = sum_sub sc_sub sum_{k in sub} (q_k - 32) y_k
// for weight rows 4G + i and activation rows 4grp + (l&15)/4. The A operand
// is q itself (0..63: no scale, no split into int8 planes); each B operand
// holds 4 activation rows x 4 sub-blocks of 16: lane column 4m + g carries
// row m's 16 values of k-slice G only when G == g (zeros otherwise, from
// bq pointing at zero bytes), so C[row][4m + g] is the sum over sub-block
// 4ks + g alone. A second MFMA with A = -32 adds -32 sum y. Each lane then
// multiplies by its sub-block's scale (24-bit products: |C| <= 16*32*127)
// and a quad sum adds the four sub-blocks; s0/s1 hold groups 0/1.
__device__ __forceinline__ void mf_block6(const MfRaw<DT_Q6_K>& r, int G, const int (&sc)[4][4],
                                          const uint8_t* bq0, const uint8_t* bq1, int (&s0)[4], int (&s1)[4]) {
    uint32_t ql[2][4], qh[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ql[h][k] = __builtin_amdgcn_alignbyte(r.ql[h][k + 1], r.ql[h][k], r.shift);
            qh[h][k] = __builtin_amdgcn_alignbyte(r.qh[h][k + 1], r.qh[h][k], r.shift);
        }
    const v4i zero = {0, 0, 0, 0}, m32 = {(int)0xE0E0E0E0, (int)0xE0E0E0E0, (int)0xE0E0E0E0, (int)0xE0E0E0E0};
#pragma unroll
    for (int i = 0; i < 4; i++) s0[i] = s1[i] = 0;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        // k = 64ks + 16G + j: ql byte 64h + 16G + j (nibble ks & 1), qh byte
        // 32h + 16(G & 1) + j (bits 2p, 2p+1), h = ks/2, p = 2(ks & 1) + G/2
        const int h = ks >> 1, p = 2 * (ks & 1) + (G >> 1);
        v4i aq;
#pragma unroll
        for (int k = 0; k < 4; k++)
            aq[k] = (int)((((ks & 1) ? (ql[h][k] >> 4) : ql[h][k]) & 0x0F0F0F0Fu) |
                          (((qh[h][k] >> (2 * p)) & 0x03030303u) << 4));
        const v4i b0 = *(const v4i*)(bq0 + 64 * ks), b1 = *(const v4i*)(bq1 + 64 * ks);
        v4i c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(aq, b0, zero, 0, 0, 0);
        v4i c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(aq, b1, zero, 0, 0, 0);
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(m32, b0, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(m32, b1, c1, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0[i] += __mul24(sc[i][ks], c0[i]);
            s1[i] += __mul24(sc[i][ks], c1[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s0[i] = quad_sum(s0[i]);
        s1[i] = quad_sum(s1[i]);
    }
}

// LDS: the waves' staging regions, the (S, M) table [nb][16][M] (int2; Q6_K int), the block scales'
// f16 bits per (block, row), dx per (block, activation row) and the
// refusal flag per (row, activation row).
template <uint32_t DT>
__host__ __device__ constexpr size_t mf_lds_bytes(int nb, int M, int nw) {
    return nw * (size_t)MfWave<DT>::LBYTES + (size_t)nb * MF_ROWS * M * (DT == DT_Q4_K ? 8 : 4) + (size_t)nb * MF_ROWS * 4 + (size_t)nb * M * 4 +
           (size_t)MF_ROWS * M * 4 * 2;  // (+ the results [16][M] for the decoder epilogues)
}

// v row `row` (kv head row / RD, dim row % RD) of activation row m into the
// value cache at the row's cache index (not stored outside the cache).
template <int RD>
__device__ __forceinline__ void mf_store_v(const MfmaArgs& A, int row, int64_t p, float v) {
    if constexpr (RD != 0) {
        if (p < 0 || p >= A.C) return;
        const int64_t at = vcache_at(row / RD, p, row % RD, RD, A.C);
        if (A.f16) ((_Float16*)A.vc)[at] = (_Float16)v;
        else ((float*)A.vc)[at] = v;
    }
}

// Workgroup `bid` of the launch's tiles of A (its 16 rows of one matrix;
// SW: rows 8 bid .. 8 bid + 7 of gate as local rows 0..7 and the same rows
// of up as local rows 8..15, swiglu of each pair in the epilogue).
template <uint32_t DT, int NW, int RD, bool SW = false>
__device__ __forceinline__ void mfma_tile(const MfmaArgs& A, int bid, uint8_t* smem) {
    static_assert(!SW || (DT == DT_Q4_K && RD == 0), "swiglu epilogue: Q4_K gate and up, no rope");
    using S = MfWave<DT>;
    constexpr int MF_T = 64 * NW;
    int mi = 0;  // (SW: mat[0], gate; up is matof's)
    if (!SW && A.nmat > 1 && bid >= A.mat[1].tile0) mi = 1;
    if (!SW && A.nmat > 2 && bid >= A.mat[2].tile0) mi = 2;
    const MfmaMat P = mi == 0 ? A.mat[0] : mi == 1 ? A.mat[1] : A.mat[2];
    const int t = threadIdx.x, l = t & 63, ar = l & 15, G = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the block loop is scalar
    const int nb = A.nb, M = A.M, N = P.N;
    const int tile = bid - P.tile0, row0 = tile * MF_ROWS;
    const bool epi = RD != 0 && P.kind != MF_PLAIN;  // a decoder epilogue (uniform)
    // local row r: its row of its matrix (clamped), the matrix, in range
    auto rowof = [&](int r) { return SW ? min(tile * 8 + (r & 7), N - 1) : min(mf_row<RD>(A, P, tile, r), N - 1); };
    auto matof = [&](int r) -> const MfmaMat& { return SW && r >= 8 ? A.mat[1] : P; };
    auto inrange = [&](int r) { return SW ? tile * 8 + (r & 7) < N : row0 + r < N; };
    constexpr int TW = DT == DT_Q4_K ? 2 : 1;  // table words per entry
    uint8_t* wl = smem + w * S::LBYTES;                               // this wave's staging
    int* tab = (int*)(smem + NW * S::LBYTES);                         // [nb][16][M][TW]
    uint32_t* dd = (uint32_t*)(tab + (size_t)nb * MF_ROWS * M * TW);  // [nb][16]
    float* dxs = (float*)(dd + (size_t)nb * MF_ROWS);                 // [nb][M]
    int* refl = (int*)(dxs + (size_t)nb * M);                         // [16][M]
    float* yres = (float*)(refl + (size_t)MF_ROWS * M);                // [16][M]: results (epilogues)

    // This lane's weight row (A operand; rows past N read the last row) and
    // activation row (B operand).
    const uint8_t* rowp = P.W + (int64_t)rowof(ar) * A.rb;
    const int am = min(ar, M - 1);
    const int8_t* yh = A.q + (int64_t)min(ar >> 1, M - 1) * A.K;  // Q4_K: the A operand's activation row
    const float* dxr = A.d32 + (int64_t)am * (A.K / 32);

    // Lane t < 16*M owns (row t/M, activation row t%M) at the end. Its
    // flags and bias are loaded first and looked at last.
    const int ft = min(t, MF_ROWS * M - 1), fr = ft / M;
    int fm = ft - fr * M;
    asm volatile("v_mov_b32 %0, %1" : "=v"(fm) : "v"(fm));  // a vector index: ok[] through the vector cache
    const int frow = rowof(fr);
    const MfmaMat& FM = matof(fr);
    const int wr = FM.wref[frow], okm = A.ok[fm];
    const float bias = FM.bias ? FM.bias[frow] : 0.f;
    const int64_t pidx = RD != 0 && P.kind != MF_PLAIN ? A.cidx[fm] : 0;  // (epilogues: cache index of row fm)
    // (rope: this lane's position and frequency, loaded before the weights)
    const bool rot_lane = RD != 0 && (P.kind == MF_ROPE_Q || P.kind == MF_ROPE_K) && t < MF_ROWS * M;
    int rot_i = 0;
    if (RD != 0) {
        const int Q = tile * 8 + (fr >> 1);
        rot_i = Q - (Q / (RD > 0 ? RD / 2 : 1)) * (RD > 0 ? RD / 2 : 1);
    }
    const bool rot_on = rot_lane && rot_i < A.rotary / 2;
    const int64_t rot_pos = rot_on ? A.pos[fm] : 0;
    const double rot_f = rot_on ? A.inv_freq[rot_i] : 0.0;

    const MfLanes<DT> L([&](int r) { return matof(r).W + (int64_t)rowof(r) * A.rb; });
    // rope: the rotation of chain lane t's (row t/M, activation row t%M),
    // computed once the first weights are requested
    float rc = 1.f, rs = 0.f;
    auto rotation = [&]() {
        if (rot_on) {
            const double ang = (double)rot_pos * rot_f;
            rc = (float)cos(ang);
            rs = (float)sin(ang);
        }
    };
    if constexpr (DT == DT_Q4_K) {
        // Block b's table entries, scale bits and dx.
        auto step = [&](const MfRaw<DT>& r, int b) {
            int s[2], mt[2];
            mf_block<DT>(r, G, ar, s, mt);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (2 * G + j < M) {
                    int* e = tab + (((size_t)b * MF_ROWS + ar) * M + 2 * G + j) * TW;
                    e[0] = s[j];
                    e[1] = mt[j];
                }
            }
            if (G == 0) dd[b * MF_ROWS + ar] = r.hdr.x;
            if (G == 1 && ar < M) dxs[b * M + ar] = r.dx;
        };
        // The activation operand (activation row ar/2, clamped) and the
        // scale of activation row ar (for the dx table) of block b.
        auto load_a = [&](int b, v4i* act, float& dx) {
            const int8_t* yb = yh + (int64_t)b * 256;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) act[ks] = *(const v4i*)(yb + 64 * ks + 16 * G);
            dx = dxr[8 * b];
        };
        // Block b: stage it, load block b + NW into the freed weight
        // registers, read the operand back, compute, then load that block's
        // activations (one block's weights in flight while one computes).
        // Every load is issued unconditionally (past the last block: the
        // last block again), so the compiler's waits before the staging
        // count exactly the loads issued after the set's.
        auto body = [&](int b, u32x4* v, v4i* act, float& dx) {
            mf_stage_w<DT>(L, wl, v);
            const int bn = min(b + NW, nb - 1);
            mf_load_w<DT>(L, bn, v);
            if (b < nb) {
                MfRaw<DT> r;
                mf_lds_w<DT>(wl + ar * (S::RST * 16), G, r);
#pragma unroll
                for (int ks = 0; ks < 4; ks++) r.act[ks] = act[ks];
                r.dx = dx;
                step(r, b);
            }
            load_a(bn, act, dx);
        };
        u32x4 v0[S::NLD];
        v4i a0[4];
        float d0;
        mf_load_w<DT>(L, min(w, nb - 1), v0);
        load_a(min(w, nb - 1), a0, d0);
        rotation();
        for (int b = w; b < nb; b += NW) body(b, v0, a0, d0);
    } else {
        uint8_t* wa = wl + S::WBYTES;    // activation rows [8][Q6_AROW]
        uint8_t* wz = wa + 8 * Q6_AROW;  // 256 zero bytes
        if (l < 16) *(u32x4*)(wz + 16 * l) = u32x4{0, 0, 0, 0};
        // The block's activations as two coalesced chunks per lane: chunk
        // c = 64i + l is row 4i + l/16 (clamped to M - 1), bytes 16(l % 16).
        const int8_t* yc0 = A.q + (int64_t)min(l >> 4, M - 1) * A.K + 16 * (l & 15);
        const int8_t* yc1 = A.q + (int64_t)min(4 + (l >> 4), M - 1) * A.K + 16 * (l & 15);
        const uint32_t ac0 = (uint32_t)(l >> 4) * Q6_AROW + 16 * (l & 15), ac1 = ac0 + 4 * Q6_AROW;
        // B operand sources: lane column 4m + g (m = (l&15)/4, g = l&3) reads
        // activation row 4grp + m, k-slice G, when G == g, else zeros.
        const int mq = (l & 15) >> 2, g = l & 3;
        const uint8_t* bq0 = G == g ? wa + mq * Q6_AROW + 16 * G : wz;
        const uint8_t* bq1 = G == g ? wa + (4 + mq) * Q6_AROW + 16 * G : wz;
        // Weight rows 4G + i of the C layout: the low 4 bits of their first
        // byte's address, for the offset of their blocks in the staging.
        uint32_t rlo[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            rlo[i] = (uint32_t)(uintptr_t)(P.W + (int64_t)rowof(4 * G + i) * A.rb) & 15;
        auto load6 = [&](int b, u32x4* v, v4i* ac, float& dx) {
            mf_load_w<DT>(L, b, v);
            ac[0] = *(const v4i*)(yc0 + (int64_t)b * 256);
            ac[1] = *(const v4i*)(yc1 + (int64_t)b * 256);
            dx = dxr[8 * b];
        };
        // Block b: stage its weights, activations and dx, load block b + NW
        // into the freed registers (in flight while this one computes; two
        // or three ahead measured slower: fewer waves fit), then compute
        // from the staging.
        auto body6 = [&](int b, u32x4* v, v4i* ac, float& dx) {
            mf_stage_w<DT>(L, wl, v);
            *(v4i*)(wa + ac0) = ac[0];
            *(v4i*)(wa + ac1) = ac[1];
            if (b < nb && G == 1 && ar < M) dxs[b * M + ar] = dx;
            load6(min(b + NW, nb - 1), v, ac, dx);
            if (b < nb) {
                MfRaw<DT> r;
                const uint32_t ob = (uint32_t)b * Q6K_BYTES;
                mf_lds_w<DT>(wl + ar * (S::RST * 16) + (((uint32_t)(uintptr_t)rowp + ob) & 15), G, r);
                if (G == 0) dd[b * MF_ROWS + ar] = r.dbits;
                int sc[4][4];  // rows 4G + i, sub-blocks 4ks + g
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint8_t* sp = wl + (4 * G + i) * (S::RST * 16) + ((rlo[i] + ob) & 15) + 192 + g;
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) sc[i][ks] = (int)*(const int8_t*)(sp + 4 * ks);
                }
                int s0[4], s1[4];
                mf_block6(r, G, sc, bq0, bq1, s0, s1);
                if (g == 0) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        int* e = tab + ((size_t)b * MF_ROWS + 4 * G + i) * M;
                        if (mq < M) e[mq] = s0[i];
                        if (4 + mq < M) e[4 + mq] = s1[i];
                    }
                }
            }
        };
        u32x4 v0[S::NLD];
        v4i c0[2];
        float d0;
        load6(min(w, nb - 1), v0, c0, d0);
        rotation();
        for (int b = w; b < nb; b += NW) body6(b, v0, c0, d0);
    }
    const int flag = (wr != 0) | (okm == 0);
    if (t < MF_ROWS * M) refl[t] = flag;
    __syncthreads();

    // The serial float chain, one lane per (weight row, activation row).
    if (t < MF_ROWS * M) {
        const int r = t / M, m = t - r * M, row = rowof(r);
        if (inrange(r) && !flag) {
            float tot = 0.f, off = 0.f;
            // (unrolled: the table reads of eight blocks are issued together,
            // so only the fma chain itself is serial)
#pragma unroll 8
            for (int b = 0; b < nb; b++) {
                const int* e = tab + (((size_t)b * MF_ROWS + r) * M + m) * TW;
                const uint32_t bits = dd[b * MF_ROWS + r];
                const float dx = dxs[b * M + m];
                tot = __builtin_fmaf((float)e[0], f16_to_f32(bits & 0xFFFFu) * dx, tot);
                if constexpr (DT == DT_Q4_K) off = __builtin_fmaf((float)e[1], f16_to_f32(bits >> 16) * dx, off);
            }
            float res = DT == DT_Q4_K ? tot - off : tot;
            if (FM.bias) res += bias;  // (FM: this lane's row's matrix, fr == r)
            if (epi && P.kind == MF_STORE_V) mf_store_v<RD>(A, row, pidx, res);
            else if (epi || SW) yres[r * M + m] = res;
            else P.y[(int64_t)m * N + row] = res;
        }
    }
    // The float32 path for refused pairs, one group of eight lanes per pair.
    const int g = t >> 3;
    for (int qq = g; qq < MF_ROWS * M; qq += MF_T / 8) {
        const int r = qq / M, m = qq - r * M, row = rowof(r);
        if (inrange(r) && refl[qq]) {
            const MfmaMat& RM = matof(r);
            float res = f32dot_g8<DT>(RM.W + (int64_t)row * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
            if (RM.bias) res += RM.bias[row];
            if ((t & 7) == 0) {
                if (epi && P.kind == MF_STORE_V) mf_store_v<RD>(A, row, A.cidx[m], res);
                else if (epi || SW) yres[qq] = res;
                else P.y[(int64_t)m * N + row] = res;
            }
        }
    }
    if constexpr (SW) {
        // every (row, activation row) result of gate and up is in yres: one lane a pair
        __syncthreads();
        if (t < 8 * M) {
            const int r = t / M, m = t - r * M, n = tile * 8 + r;
            const int64_t i = (int64_t)m * N + n;
            if (n < N) A.sw[i] = swiglu_at(yres[r * M + m], yres[(r + 8) * M + m], i, A.sw_total, A.sw_chunk);
        }
    }
    if constexpr (RD != 0) {
        if (!epi || P.kind == MF_STORE_V) return;
        // every (row, activation row) result of q or k is in yres: one lane each
        __syncthreads();
        if (t < MF_ROWS * M) {
            const int r = t / M, m = t - r * M, row = rowof(r);
            const int64_t p = pidx;  // (t < 16 M: the cache index of row m)
            float own = yres[t];
            {
                // rope_kv_kernel's steps on (dim a, dim b) = rows (2j, 2j+1)
                const float other = yres[(r ^ 1) * M + m];
                const int Q = tile * 8 + (r >> 1), hh = Q / (RD / 2), i = Q - hh * (RD / 2);
                float o = own;
                if (i < A.rotary / 2) {
                    const float x1 = (r & 1) ? other : own, x2 = (r & 1) ? own : other;
                    o = (r & 1) ? x2 * rc + x1 * rs : x1 * rc - x2 * rs;
                }
                if (P.kind == MF_ROPE_Q) {
                    P.y[(int64_t)m * N + row] = o;
                } else if (p >= 0 && p < A.C) {
                    const int64_t at = ((int64_t)hh * A.C + p) * RD + (row - hh * RD);
                    if (A.f16) ((_Float16*)A.kc)[at] = (_Float16)o;
                    else ((float*)A.kc)[at] = o;
                }
            }
        }
    }
}

// Q4_K fits 5 waves per SIMD (at most 102 registers) with one block ahead.
template <uint32_t DT, int NW, int RD = 0, bool SW = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(DT == DT_Q4_K ? 5 : 1)))
void gemv_a8k_mfma_kernel(MfmaArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    mfma_tile<DT, NW, RD, SW>(A, (int)blockIdx.x, smem);
}

// q and k (rope; k to the key cache) and v (to the value cache) in one
// launch: workgroups below `split` take QK's tiles, the others V's, four
// waves each. Both parts are latency-bound on their own (8B at 8 rows: q+k
// 320 workgroups, v 64), so one launch saves the second one's ramp and drain.
template <uint32_t DT0, uint32_t DT1, int RD>
__global__ __launch_bounds__(256) void gemv_a8k_mfma_qkv_kernel(MfmaArgs QK, MfmaArgs V, int split) {
    extern __shared__ __align__(16) uint8_t smem[];
    if ((int)blockIdx.x < split) mfma_tile<DT0, 4, RD>(QK, (int)blockIdx.x, smem);
    else mfma_tile<DT1, 4, RD>(V, (int)blockIdx.x - split, smem);
}

// Waves per workgroup: 4, or for Q6_K 12 while the grid holds fewer than
// 4096 waves (16 per CU) and K has 16 blocks or more, else 8. Measured at
// the llama-8B shapes and 8 rows: Q4_K is fastest at 4 whatever the grid
// (gate+up 22.5 us at 4, 28.6 at 8, 39 at 16); Q6_K down 17.5 us at 12,
// 17.9 at 8, 18.4 at 16 (which spills: 128 registers per lane).
static int mf_waves(uint32_t dt, int64_t tiles, int nb) {
    if (dt == DT_Q6_K && tiles * 4 < 4096 && nb >= 8) return nb >= 16 ? 12 : 8;
    return 4;
}

static size_t mf_lds(uint32_t dt, int nb, int M, int nw) {
    return dt == DT_Q4_K ? mf_lds_bytes<DT_Q4_K>(nb, M, nw) : mf_lds_bytes<DT_Q6_K>(nb, M, nw);
}

bool gemv_mfma_ok(const DevWeight* const* ws, int nmat, int64_t rows) {
    if (rows < 2 || rows > 8 || nmat < 1 || nmat > 3) return false;
    const DevWeight& w = *ws[0];
    if ((w.dt != DT_Q4_K && w.dt != DT_Q6_K) || w.k % 256 || w.k <= 0) return false;
    int64_t tiles = 0;
    for (int i = 0; i < nmat; i++) {
        if (ws[i]->dt != w.dt || ws[i]->k != w.k || ws[i]->n <= 0) return false;
        tiles += (ws[i]->n + MF_ROWS - 1) / MF_ROWS;
    }
    const int nb = (int)(w.k / 256);
    return mf_lds(w.dt, nb, (int)rows, mf_waves(w.dt, tiles, nb)) <= 160 * 1024;  // gfx950: 160 KB of LDS per workgroup
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
        A.mat[i].kind = MF_PLAIN;
        if (i < nmat) tiles += (int)((wi.n + MF_ROWS - 1) / MF_ROWS);
    }
    A.pos = A.cidx = nullptr;
    A.inv_freq = nullptr;
    A.rotary = A.interleaved = A.f16 = 0;
    A.C = 0;
    A.kc = A.vc = nullptr;
    A.sw = nullptr;
    A.sw_total = A.sw_chunk = 0;
    const int nw = mf_waves(w.dt, tiles, A.nb);
    const size_t lds = mf_lds(w.dt, A.nb, A.M, nw);
    const dim3 grid((unsigned)tiles), block((unsigned)(64 * nw));
    if (w.dt == DT_Q4_K) {
        hipLaunchKernelGGL((gemv_a8k_mfma_kernel<DT_Q4_K, 4>), grid, block, lds, stream, A);
    } else {
        if (nw == 4) hipLaunchKernelGGL((gemv_a8k_mfma_kernel<DT_Q6_K, 4>), grid, block, lds, stream, A);
        else if (nw == 8) hipLaunchKernelGGL((gemv_a8k_mfma_kernel<DT_Q6_K, 8>), grid, block, lds, stream, A);
        else hipLaunchKernelGGL((gemv_a8k_mfma_kernel<DT_Q6_K, 12>), grid, block, lds, stream, A);
    }
    return hipGetLastError();
}

// gate and up at 2..8 activation rows with swiglu in the epilogue (Q4_K,
// N % 8 == 0): a workgroup per 8 rows of each, four waves.
bool gemv_mfma_swiglu_ok(const DevWeight& gate, const DevWeight& up, int64_t rows) {
    if (rows < 2 || rows > 8) return false;
    if (gate.dt != DT_Q4_K || up.dt != DT_Q4_K || gate.n != up.n || gate.k != up.k || gate.k % 256 ||
        gate.k <= 0 || gate.n % 8 || gate.n > (1 << 30))
        return false;
    return mf_lds(DT_Q4_K, (int)(gate.k / 256), (int)rows, 4) <= 160 * 1024;
}

hipError_t launch_gemv_a8k_mfma_swiglu(const DevWeight& gate, const DevWeight& up, const ActPtrs& a, int64_t rows,
                                       const float* x, const float* const* bias, float* out, int64_t total,
                                       int64_t chunk, hipStream_t stream) {
    if (!gemv_mfma_swiglu_ok(gate, up, rows)) return hipErrorInvalidValue;
    MfmaArgs A;
    A.nmat = 2;
    A.rb = gate.row_bytes;
    A.nb = (int)(gate.k / 256);
    A.M = (int)rows;
    A.K = gate.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.ok = a.ok;
    A.x = x;
    A.fused = 1;  // (the call's rows are all of it: at most 8)
    const DevWeight* gu[3] = {&gate, &up, &up};
    for (int i = 0; i < 3; i++) {
        A.mat[i].W = gu[i]->data;
        A.mat[i].wref = gu[i]->wref;
        A.mat[i].bias = i < 2 && bias ? bias[i] : nullptr;
        A.mat[i].y = nullptr;
        A.mat[i].N = (int)gu[i]->n;
        A.mat[i].tile0 = 0;
        A.mat[i].kind = MF_PLAIN;
    }
    A.pos = A.cidx = nullptr;
    A.inv_freq = nullptr;
    A.rotary = A.interleaved = A.f16 = 0;
    A.C = 0;
    A.kc = A.vc = nullptr;
    A.sw = out;
    A.sw_total = total;
    A.sw_chunk = chunk;
    const size_t lds = mf_lds(DT_Q4_K, A.nb, A.M, 4);
    hipLaunchKernelGGL((gemv_a8k_mfma_kernel<DT_Q4_K, 4, 0, true>), dim3((unsigned)(gate.n / 8)), dim3(256), lds,
                       stream, A);
    return hipGetLastError();
}

// q, k (rope) and v (cache scatter) at 2..8 activation rows: one launch.
bool gemv_mfma_qkv_ok(const DevWeight* const* ws, int64_t rows, int heads, int kv_heads, int d, int rotary) {
    if ((d != 64 && d != 128) || rotary <= 0 || rotary % 2 || rotary > d) return false;
    if (ws[0]->n != (int64_t)heads * d || ws[1]->n != (int64_t)kv_heads * d || ws[2]->n != (int64_t)kv_heads * d)
        return false;
    return gemv_mfma_ok(ws, 2, rows) && gemv_mfma_ok(ws + 2, 1, rows);
}

// Sets the parts' first tiles; returns the launch's tile count.
static int mf_tiles(MfmaArgs& A) {
    int tiles = 0;
    for (int i = 0; i < A.nmat; i++) {
        A.mat[i].tile0 = tiles;
        tiles += (A.mat[i].N + MF_ROWS - 1) / MF_ROWS;
    }
    return tiles;
}

template <int RD>
static hipError_t launch_mfma_qkv(MfmaArgs QK, MfmaArgs V, uint32_t dt0, uint32_t dt1, hipStream_t stream) {
    const int split = mf_tiles(QK), tiles = split + mf_tiles(V);
    const size_t lds = std::max(mf_lds(dt0, QK.nb, QK.M, 4), mf_lds(dt1, V.nb, V.M, 4));
    const dim3 grid((unsigned)tiles), block(256);
    if (dt0 == DT_Q4_K && dt1 == DT_Q4_K)
        hipLaunchKernelGGL((gemv_a8k_mfma_qkv_kernel<DT_Q4_K, DT_Q4_K, RD>), grid, block, lds, stream, QK, V, split);
    else if (dt0 == DT_Q4_K)
        hipLaunchKernelGGL((gemv_a8k_mfma_qkv_kernel<DT_Q4_K, DT_Q6_K, RD>), grid, block, lds, stream, QK, V, split);
    else if (dt1 == DT_Q4_K)
        hipLaunchKernelGGL((gemv_a8k_mfma_qkv_kernel<DT_Q6_K, DT_Q4_K, RD>), grid, block, lds, stream, QK, V, split);
    else
        hipLaunchKernelGGL((gemv_a8k_mfma_qkv_kernel<DT_Q6_K, DT_Q6_K, RD>), grid, block, lds, stream, QK, V, split);
    return hipGetLastError();
}

hipError_t launch_gemv_a8k_mfma_qkv(const DevWeight* const* ws, const ActPtrs& a, int64_t rows, const float* x,
                                    const float* const* bias, float* q, const int64_t* pos, const int64_t* cidx,
                                    const double* inv_freq, int heads, int kv_heads, int d, int rotary,
                                    int interleaved, int64_t context, void* kc, void* vc, int f16,
                                    hipStream_t stream) {
    if (!gemv_mfma_qkv_ok(ws, rows, heads, kv_heads, d, rotary)) return hipErrorInvalidValue;
    MfmaArgs AP[2];
    for (int part = 0; part < 2; part++) {
        const int nmat = part == 0 ? 2 : 1;
        const DevWeight* const* wp = ws + (part == 0 ? 0 : 2);
        MfmaArgs& A = AP[part];
        A.nmat = nmat;
        A.rb = wp[0]->row_bytes;
        A.nb = (int)(wp[0]->k / 256);
        A.M = (int)rows;
        A.K = wp[0]->k;
        A.q = a.q;
        A.d32 = a.d32;
        A.ok = a.ok;
        A.x = x;
        A.fused = rows <= 8;
        for (int i = 0; i < 3; i++) {
            const DevWeight& wi = *wp[i < nmat ? i : 0];
            A.mat[i].W = wi.data;
            A.mat[i].wref = wi.wref;
            A.mat[i].bias = i < nmat && bias ? bias[(part == 0 ? 0 : 2) + i] : nullptr;
            A.mat[i].y = part == 0 && i == 0 ? q : nullptr;
            A.mat[i].N = (int)wi.n;
            A.mat[i].tile0 = 0;
            A.mat[i].kind = part == 1 ? MF_STORE_V : i == 0 ? MF_ROPE_Q : MF_ROPE_K;
        }
        A.pos = pos;
        A.cidx = cidx;
        A.inv_freq = inv_freq;
        A.rotary = rotary;
        A.interleaved = interleaved;
        A.f16 = f16;
        A.C = context;
        A.kc = kc;
        A.vc = vc;
        A.sw = nullptr;
        A.sw_total = A.sw_chunk = 0;
    }
    return d == 64 ? launch_mfma_qkv<64>(AP[0], AP[1], ws[0]->dt, ws[2]->dt, stream)
                   : launch_mfma_qkv<128>(AP[0], AP[1], ws[0]->dt, ws[2]->dt, stream);
}

}  // namespace mimg
