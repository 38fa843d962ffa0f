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
// Two kernels compute the same bits:
//
// gemv_a8k_pairs_kernel (the default): a 256-thread workgroup owns R weight
// rows. Its 32 groups of 8 lanes take the R*nb (row, block) pairs in turn,
// U pairs at a time with all their weight loads issued before any compute,
// so that many 128-bit loads per lane are in flight (the GEMV is bound by
// HBM latency x bandwidth). For a pair, lane l of the group loads 16 bytes
// of the block's quants, forms its part of S with v_dot4_i32_i8 against the
// activation quants (read through L1, they are shared by all rows), and the
// group sums the parts with three DPP steps (integer, so exact in any
// order). The exact (S, M) and the two f32 scale products of every pair go
// to LDS; then one lane per (row, activation row) runs the serial float
// chain over the blocks in order.
//
// gemv_a8k_tiled_kernel: a group of 8 lanes owns one weight row and walks
// its blocks in order, with the activation quants of up to 8 rows staged in
// LDS in tiles of blocks.
//
// Rows of x the quantizer refused and rows of w with a non-finite block scale
// take the float32 path (reference linearA8, interp/fast.go:323-377), in the
// reference's AVX2 order (f32path.hpp).
#include <cstdlib>

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
__global__ __launch_bounds__(256) void gemv_a8k_tiled_kernel(GemvArgs A) {
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

// One lane's share of a Q4_K block: lane l holds quant bytes 16l..16l+15 of
// the block, i.e. chunk c = l/2, elements 64c+16h+[0,16) (low nibbles,
// sub-block 2c) and 64c+32+16h+[0,16) (high nibbles, sub-block 2c+1), with
// h = l%2; for the M term it takes sub-block l.
struct Q4KLane {
    uint32_t lo[4], hi[4];
    int scl, sch, mm, yoff;
    float d, dmin;
};

__device__ __forceinline__ Q4KLane q4k_lane(const u32x4& hdr, const u32x4& qv, int l) {
    Q4KLane w;
    const Q4KScales s = q4k_scales(hdr.y, hdr.z, hdr.w);
    const int c = l >> 1, h = l & 1;
    w.scl = (int)byte_of(s.sc, 2 * c);
    w.sch = (int)byte_of(s.sc, 2 * c + 1);
    w.mm = (int)byte_of(s.m, l);
    w.d = f16_to_f32(hdr.x & 0xFFFFu);
    w.dmin = f16_to_f32(hdr.x >> 16);
    w.yoff = 64 * c + 16 * h;
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w.lo[k] = q[k] & 0x0F0F0F0Fu;
        w.hi[k] = (q[k] >> 4) & 0x0F0F0F0Fu;
    }
    return w;
}

// The lane's part of S: sc_2c * sum(lo*y) + sc_2c+1 * sum(hi*y) (exact).
__device__ __forceinline__ int q4k_part(const Q4KLane& w, const u32x4& ya, const u32x4& yh) {
    int dl = sdot4(w.lo[0], ya.x, 0);
    dl = sdot4(w.lo[1], ya.y, dl);
    dl = sdot4(w.lo[2], ya.z, dl);
    dl = sdot4(w.lo[3], ya.w, dl);
    int dh = sdot4(w.hi[0], yh.x, 0);
    dh = sdot4(w.hi[1], yh.y, dh);
    dh = sdot4(w.hi[2], yh.z, dh);
    dh = sdot4(w.hi[3], yh.w, dh);
    return w.scl * dl + w.sch * dh;
}

// Raw loads of one lane's share of a Q6_K block (2-byte aligned blocks):
// lane l = 4h + p takes ql bytes 64h+16p..+16 (elements eL..eL+15 in their
// low nibbles and eH = eL+64.. in their high nibbles, eL = 128h+32(p/2)+16(p%2)),
// the qh bytes 32h+16(p%2)..+16 and the block's scales and d.
struct Q6KRaw {
    u32x4 ql, qh;
    uint32_t sw0, sw1, dbits;
};

__device__ __forceinline__ Q6KRaw q6k_load(const uint8_t* blk, int l) {
    const int h = l >> 2, p = l & 3;
    Q6KRaw r;
    r.ql = load16_a2(blk + 64 * h + 16 * p);
    r.qh = load16_a2(blk + 128 + 32 * h + 16 * (p & 1));
    r.sw0 = load4_a2(blk + 192 + 8 * h);
    r.sw1 = load4_a2(blk + 196 + 8 * h);
    r.dbits = load_u16(blk + 208);
    return r;
}

struct Q6KLane {
    uint32_t vl[4], vh[4];
    int scl, sch, eL;
    float d;
};

__device__ __forceinline__ Q6KLane q6k_lane(const Q6KRaw& r, int l) {
    const int h = l >> 2, p = l & 3, pp = p >> 1, p1 = p & 1;
    Q6KLane w;
    const int idx = 2 * pp + p1;
    w.scl = (int)(int8_t)(r.sw0 >> (8 * idx));
    w.sch = (int)(int8_t)(r.sw1 >> (8 * idx));
    w.d = f16_to_f32(r.dbits);
    w.eL = 128 * h + 32 * pp + 16 * p1;
    const int shL = 2 * pp, shH = 4 + 2 * pp;
    const uint32_t qlw[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
    const uint32_t qhw[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w.vl[k] = (qlw[k] & 0x0F0F0F0Fu) | (((qhw[k] >> shL) & 0x03030303u) << 4);
        w.vh[k] = ((qlw[k] >> 4) & 0x0F0F0F0Fu) | (((qhw[k] >> shH) & 0x03030303u) << 4);
    }
    return w;
}

// The lane's part of S: sc_L*(sum(q*y) - 32*sum(y)) + sc_H*(...) over its
// two runs of 16 (exact); ysL/ysH are the runs' activation sums.
__device__ __forceinline__ int q6k_part(const Q6KLane& w, const u32x4& ya, const u32x4& yh, int ysL, int ysH) {
    int dl = sdot4(w.vl[0], ya.x, 0);
    dl = sdot4(w.vl[1], ya.y, dl);
    dl = sdot4(w.vl[2], ya.z, dl);
    dl = sdot4(w.vl[3], ya.w, dl);
    int dh = sdot4(w.vh[0], yh.x, 0);
    dh = sdot4(w.vh[1], yh.y, dh);
    dh = sdot4(w.vh[2], yh.z, dh);
    dh = sdot4(w.vh[3], yh.w, dh);
    return w.scl * (dl - 32 * ysL) + w.sch * (dh - 32 * ysH);
}

template <uint32_t DT, int M, int R>
__global__ __launch_bounds__(256) void gemv_a8k_pairs_kernel(GemvArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    i32x4* part = (i32x4*)smem;  // [R][nb][M]: S, M term, bits(d*dx), bits(dmin*dx)
    constexpr int U = 4;
    const int g = threadIdx.x >> 3, l = threadIdx.x & 7;
    const int nb = A.nb, row0 = blockIdx.x * R, npairs = R * nb;
    const int64_t K = A.K, R32 = K / 32, R16 = K / 16;

    for (int p0 = g; p0 < npairs; p0 += 32 * U) {
        if (DT == DT_Q4_K) {
            u32x4 hdr[U], qv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + 32 * u;
                if (p < npairs) {
                    const int r = p / nb, b = p - r * nb;
                    const int row = min(row0 + r, A.N - 1);
                    const uint8_t* blk = A.W + (int64_t)row * A.rb + (int64_t)b * Q4K_BYTES;
                    hdr[u] = *(const u32x4*)blk;
                    qv[u] = *(const u32x4*)(blk + 16 + 16 * l);
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + 32 * u;
                if (p >= npairs) break;  // uniform within the group
                const int r = p / nb, b = p - r * nb;
                const Q4KLane w = q4k_lane(hdr[u], qv[u], l);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const int8_t* yb = A.q + m * K + (int64_t)b * 256 + w.yoff;
                    const u32x4 ya = *(const u32x4*)yb;
                    const u32x4 yh = *(const u32x4*)(yb + 32);
                    const int S = group8_sum(q4k_part(w, ya, yh));
                    const int Mt = group8_sum(w.mm * (int)A.s16[m * R32 + 8 * b + l]);
                    const float dx = A.d32[m * R32 + 8 * b];
                    if (l == 0) {
                        i32x4 v;
                        v.x = S;
                        v.y = Mt;
                        v.z = __float_as_int(w.d * dx);
                        v.w = __float_as_int(w.dmin * dx);
                        part[(r * nb + b) * M + m] = v;
                    }
                }
            }
        } else {
            Q6KRaw raw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + 32 * u;
                if (p < npairs) {
                    const int r = p / nb, b = p - r * nb;
                    const int row = min(row0 + r, A.N - 1);
                    raw[u] = q6k_load(A.W + (int64_t)row * A.rb + (int64_t)b * Q6K_BYTES, l);
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + 32 * u;
                if (p >= npairs) break;
                const int r = p / nb, b = p - r * nb;
                const Q6KLane w = q6k_lane(raw[u], l);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const int8_t* yb = A.q + m * K + (int64_t)b * 256;
                    const u32x4 ya = *(const u32x4*)(yb + w.eL);
                    const u32x4 yh = *(const u32x4*)(yb + w.eL + 64);
                    const int16_t* ys = A.s16 + m * R16 + 16 * b;
                    const int S = group8_sum(q6k_part(w, ya, yh, ys[w.eL >> 4], ys[(w.eL + 64) >> 4]));
                    const float dx = A.d32[m * R32 + 8 * b];
                    if (l == 0) {
                        i32x4 v;
                        v.x = S;
                        v.y = 0;
                        v.z = __float_as_int(w.d * dx);
                        v.w = 0;
                        part[(r * nb + b) * M + m] = v;
                    }
                }
            }
        }
    }
    __syncthreads();

    // The serial float chain, one lane per (weight row, activation row).
    const int t = threadIdx.x;
    if (t < R * M) {
        const int r = t / M, m = t - r * M, row = row0 + r;
        if (row < A.N && A.wref[row] == 0 && A.ok[m]) {
            float tot = 0.f, off = 0.f;
            for (int b = 0; b < nb; b++) {
                const i32x4 v = part[(r * nb + b) * M + m];
                tot = __builtin_fmaf((float)v.x, __int_as_float(v.z), tot);
                if (DT == DT_Q4_K) off = __builtin_fmaf((float)v.y, __int_as_float(v.w), off);
            }
            float res = DT == DT_Q4_K ? tot - off : tot;
            if (A.bias) res += A.bias[row];
            A.y[(int64_t)m * A.y_stride + row] = res;
        }
    }
    // The float32 path for refused pairs, one group of eight lanes per pair.
    for (int qq = g; qq < R * M; qq += 32) {
        const int r = qq / M, m = qq - r * M, row = row0 + r;
        if (row < A.N && (A.wref[row] != 0 || !A.ok[m])) {
            float res = f32dot_g8<DT>(A.W + (int64_t)row * A.rb, A.x + (int64_t)m * K, K, A.fused != 0);
            if (A.bias) res += A.bias[row];
            if (l == 0) A.y[(int64_t)m * A.y_stride + row] = res;
        }
    }
}

// Kernel choice: 0 = pairs (default), 1 = tiled. MIMG_GEMV_VARIANT selects
// the other for A/B timing; both give the same bits.
static int gemv_variant() {
    static const int v = [] {
        const char* e = getenv("MIMG_GEMV_VARIANT");
        return e ? atoi(e) : 0;
    }();
    return v;
}

template <uint32_t DT, int M, int R>
static hipError_t launch_pairs_r(GemvArgs A, hipStream_t stream) {
    const size_t lds = (size_t)R * A.nb * M * 16;
    dim3 grid((unsigned)((A.N + R - 1) / R)), blk(256);
    hipLaunchKernelGGL((gemv_a8k_pairs_kernel<DT, M, R>), grid, blk, lds, stream, A);
    return hipGetLastError();
}

// Rows per workgroup: enough (row, block) pairs to keep 32 groups busy, as
// many workgroups as possible, and the pair table within 48 KB of LDS.
static int pairs_rows(int N, int nb, int M) {
    int R = 8;
    while (R > 1 && ((N + R - 1) / R < 1024 || (size_t)R * nb * M * 16 > 48 * 1024)) R >>= 1;
    return R;
}

template <uint32_t DT, int M>
static hipError_t launch_pairs(GemvArgs A, hipStream_t stream) {
    switch (pairs_rows(A.N, A.nb, M)) {
    case 8: return launch_pairs_r<DT, M, 8>(A, stream);
    case 4: return launch_pairs_r<DT, M, 4>(A, stream);
    case 2: return launch_pairs_r<DT, M, 2>(A, stream);
    default: return launch_pairs_r<DT, M, 1>(A, stream);
    }
}

template <uint32_t DT, int M>
static hipError_t launch_m(GemvArgs A, hipStream_t stream) {
    if (gemv_variant() == 0 && (size_t)A.nb * M * 16 <= 48 * 1024) return launch_pairs<DT, M>(A, stream);
    A.tb = min(A.nb, max(1, 128 / M));
    const size_t lds = (size_t)M * A.tb * (256 + 4 + 2 * KQ<DT>::S16PB);
    dim3 grid((unsigned)((A.N + 31) / 32)), blk(256);
    hipLaunchKernelGGL((gemv_a8k_tiled_kernel<DT, M>), grid, blk, lds, stream, A);
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
