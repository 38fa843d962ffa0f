// Decode GEMV, Q4_K / Q6_K weights x 8-bit activations in blocks of 256
// (dequant_matmul_a8.v2 with block = 256, the path mim-import writes for
// K-quant weights, reference importer/llama.go:264-280), for up to 8
// activation rows already quantized (quantize_act.hip).
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
// Mapping: a 256-thread workgroup owns R weight rows. Its 32 groups of 8
// lanes take the R*nb (row, block) pairs, U pairs at a time with all their
// weight loads issued before any compute, so that many 128-bit loads per
// lane are in flight (the GEMV is bound by HBM latency x bandwidth). For a
// pair, lane l of the group loads 16 bytes of the block's quants, forms its
// part of S with v_dot4_i32_i8 against the activation quants (read through
// L1, they are shared by all rows), and the group sums the parts with three
// DPP steps (integer, so exact in any order). The exact (S, M) and the two
// f32 scale products of every pair go to LDS; then one lane per (row,
// activation row) runs the serial float chain over the blocks in order.
// (A tiled kernel walking each row's blocks in order, and a persistent
// software-pipelined variant, measured slower on MI355X at these shapes.)
//
// Rows of x the quantizer refused and rows of w with a non-finite block scale
// take the float32 path (reference linearA8, interp/fast.go:323-377), in the
// reference's AVX2 order (f32path.hpp).
#include "f32path.hpp"
#include "kquant_lane.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// One matrix of a launch (up to three share the activations).
struct PairMat {
    const uint8_t* W;
    const uint8_t* wref;
    const float* bias;
    float* y;
    int N;
    int tile0;  // first workgroup of this matrix
};

struct GemvArgs {
    const uint8_t* W;
    int64_t rb;      // bytes per weight row (the same for every matrix)
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
    int fused;            // float32 fallback order: total rows <= 8
    PairMat mat[3];
    int nmat;
};

template <uint32_t DT>
struct KQ {
    static constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    static constexpr int S16PB = DT == DT_Q4_K ? 8 : 16;  // s16 entries per block
};

// Activation staging: with one activation row and K <= STAGE_MAXK the
// workgroup copies the row's quants, block sums and scales into LDS behind
// the pair table before computing, so the compute phase reads no global
// memory (global reads issued after the weight loads would wait for all of
// them, the load counter being in order).
constexpr int STAGE_MAXK = 16384;

template <uint32_t DT, int M, int R, bool STAGE>
__global__ __launch_bounds__(256) void gemv_a8k_pairs_kernel(GemvArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    i32x4* part = (i32x4*)smem;  // [R][nb][M]: S, M term, bits(d*dx), bits(dmin*dx)
    constexpr int U = 4;
    constexpr int S16PB = KQ<DT>::S16PB;
    static_assert(!STAGE || M == 1, "staging holds one activation row");
    // This workgroup's matrix of the launch.
    int mi = 0;
    if (A.nmat > 1 && (int)blockIdx.x >= A.mat[1].tile0) mi = 1;
    if (A.nmat > 2 && (int)blockIdx.x >= A.mat[2].tile0) mi = 2;
    const PairMat P = mi == 0 ? A.mat[0] : mi == 1 ? A.mat[1] : A.mat[2];
    A.W = P.W;
    A.wref = P.wref;
    A.bias = P.bias;
    A.y = P.y;
    A.N = P.N;
    A.y_stride = P.N;
    const int g = threadIdx.x >> 3, l = threadIdx.x & 7, t = threadIdx.x;
    const int nb = A.nb, row0 = ((int)blockIdx.x - P.tile0) * R, npairs = R * nb;
    const int64_t K = A.K, R32 = K / 32, R16 = K / 16;

    // Staged row: q [K] int8, s16 [nb*S16PB] int16, dx [nb] f32.
    int8_t* sq = (int8_t*)(smem + (size_t)R * nb * M * 16);
    int16_t* ss = (int16_t*)(sq + K);
    float* sdx = (float*)(ss + nb * S16PB);
    const int nq = (int)(K / 16), ns = nb * S16PB / 8;
    if constexpr (STAGE) {
        // Straight into LDS (global_load_lds: lane i of a wave writes
        // bytes [16i, 16i+16) after the wave's base), no registers held.
        const int wave = t >> 6;
#pragma unroll
        for (int j = 0; j < STAGE_MAXK / 16 / 256; j++)
            if (t + 256 * j < nq)
                __builtin_amdgcn_global_load_lds((const u32x4*)A.q + t + 256 * j,
                                                 (__attribute__((address_space(3))) void*)(sq + 1024 * wave + 4096 * j),
                                                 16, 0, 0);
        if (t < ns)
            __builtin_amdgcn_global_load_lds((const u32x4*)A.s16 + t,
                                             (__attribute__((address_space(3))) void*)((uint8_t*)ss + 1024 * wave), 16, 0, 0);
        if (t < nb)
            __builtin_amdgcn_global_load_lds(A.d32 + 8 * t, (__attribute__((address_space(3))) void*)(sdx + 64 * wave),
                                             4, 0, 0);
    }

    // With staging the loop's trip count is the same for every group (the
    // staging barrier sits in its first iteration).
    const int pstart = STAGE ? 0 : g, poff = STAGE ? g : 0;
    for (int p0 = pstart; p0 < npairs; p0 += 32 * U) {
        // The weights of this group's next U pairs, all in flight.
        u32x4 hdr[U], qv[U];
        Q6KRaw raw[U];
        // Unconditional (clamped) loads in straight-line code: a load in a
        // conditional block makes the compiler wait for every earlier load
        // before it (the blocks reuse registers), which would put the U
        // pairs' HBM round trips in series.
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int p = min(p0 + poff + 32 * u, npairs - 1);
            const int r = p / nb, b = p - r * nb;
            const int row = min(row0 + r, A.N - 1);
            const uint8_t* blk = A.W + (int64_t)row * A.rb + (int64_t)b * KQ<DT>::BYTES;
            if constexpr (DT == DT_Q4_K) {
                hdr[u] = *(const u32x4*)blk;
                qv[u] = *(const u32x4*)(blk + 16 + 16 * l);
            } else {
                raw[u] = q6k_load(blk, l);
            }
        }
        if constexpr (STAGE) {
            if (p0 == 0) {
                // The staged row and this wave's first weights have landed.
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            // Every loaded pair is consumed (a clamped duplicate past the end
            // is computed and not stored), so no load is left pending across
            // the loop's back edge, which would again cost a full wait.
            const int pu = p0 + poff + 32 * u;
            const bool store = pu < npairs;
            const int p = min(pu, npairs - 1);
            const int r = p / nb, b = p - r * nb;
            if constexpr (DT == DT_Q4_K) {
                const Q4KLane w = q4k_lane(hdr[u], qv[u], l);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    u32x4 ya, yh;
                    int xs;
                    float dx;
                    if constexpr (STAGE) {
                        const int8_t* yb = sq + 256 * b + w.yoff;
                        ya = *(const u32x4*)yb;
                        yh = *(const u32x4*)(yb + 32);
                        xs = ss[8 * b + l];
                        dx = sdx[b];
                    } else {
                        const int8_t* yb = A.q + m * K + (int64_t)b * 256 + w.yoff;
                        ya = *(const u32x4*)yb;
                        yh = *(const u32x4*)(yb + 32);
                        xs = A.s16[m * R32 + 8 * b + l];
                        dx = A.d32[m * R32 + 8 * b];
                    }
                    const int S = group8_sum(q4k_part(w, ya, yh));
                    const int Mt = group8_sum(w.mm * xs);
                    if (l == 0 && store) {
                        i32x4 v;
                        v.x = S;
                        v.y = Mt;
                        v.z = __float_as_int(w.d * dx);
                        v.w = __float_as_int(w.dmin * dx);
                        part[(r * nb + b) * M + m] = v;
                    }
                }
            } else {
                const Q6KLane w = q6k_lane(raw[u], l);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    u32x4 ya, yh;
                    int ysL, ysH;
                    float dx;
                    if constexpr (STAGE) {
                        const int8_t* yb = sq + 256 * b;
                        ya = *(const u32x4*)(yb + w.eL);
                        yh = *(const u32x4*)(yb + w.eL + 64);
                        ysL = ss[16 * b + (w.eL >> 4)];
                        ysH = ss[16 * b + ((w.eL + 64) >> 4)];
                        dx = sdx[b];
                    } else {
                        const int8_t* yb = A.q + m * K + (int64_t)b * 256;
                        ya = *(const u32x4*)(yb + w.eL);
                        yh = *(const u32x4*)(yb + w.eL + 64);
                        const int16_t* ys = A.s16 + m * R16 + 16 * b;
                        ysL = ys[w.eL >> 4];
                        ysH = ys[(w.eL + 64) >> 4];
                        dx = A.d32[m * R32 + 8 * b];
                    }
                    const int S = group8_sum(q6k_part(w, ya, yh, ysL, ysH));
                    if (l == 0 && store) {
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

template <uint32_t DT, int M, int R>
static hipError_t launch_pairs_r(GemvArgs A, hipStream_t stream) {
    int tiles = 0;
    for (int i = 0; i < A.nmat; i++) {
        A.mat[i].tile0 = tiles;
        tiles += (A.mat[i].N + R - 1) / R;
    }
    size_t lds = (size_t)R * A.nb * M * 16;
    if constexpr (M == 1) {
        if (A.K <= STAGE_MAXK) {
            lds += (size_t)A.K + (size_t)A.nb * KQ<DT>::S16PB * 2 + (size_t)A.nb * 4;
            hipLaunchKernelGGL((gemv_a8k_pairs_kernel<DT, M, R, true>), dim3((unsigned)tiles), dim3(256), lds,
                               stream, A);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_a8k_pairs_kernel<DT, M, R, false>), dim3((unsigned)tiles), dim3(256), lds, stream, A);
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
    int total_n = 0;
    for (int i = 0; i < A.nmat; i++) total_n += A.mat[i].N;
    switch (pairs_rows(total_n, A.nb, M)) {
    case 8: return launch_pairs_r<DT, M, 8>(A, stream);
    case 4: return launch_pairs_r<DT, M, 4>(A, stream);
    case 2: return launch_pairs_r<DT, M, 2>(A, stream);
    default: return launch_pairs_r<DT, M, 1>(A, stream);
    }
}

template <uint32_t DT>
static hipError_t launch_dt(GemvArgs A, int rows, hipStream_t stream) {
    switch (rows) {
    case 1: return launch_pairs<DT, 1>(A, stream);
    case 2: return launch_pairs<DT, 2>(A, stream);
    case 3: return launch_pairs<DT, 3>(A, stream);
    case 4: return launch_pairs<DT, 4>(A, stream);
    case 5: return launch_pairs<DT, 5>(A, stream);
    case 6: return launch_pairs<DT, 6>(A, stream);
    case 7: return launch_pairs<DT, 7>(A, stream);
    case 8: return launch_pairs<DT, 8>(A, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_a8k(const DevWeight* const* ws, int nmat, const ActPtrs& a, int64_t rows,
                           int64_t total_rows, const float* x, const float* const* bias, float* const* y,
                           hipStream_t stream) {
    if (rows < 1 || rows > 8 || nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    const DevWeight& w = *ws[0];
    for (int i = 0; i < nmat; i++)
        if (ws[i]->dt != w.dt || ws[i]->k != w.k || ws[i]->n <= 0) return hipErrorInvalidValue;
    if (w.k % 256) return hipErrorInvalidValue;
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
    A.bias = nullptr;
    A.y = nullptr;
    A.y_stride = w.n;
    A.fused = total_rows <= 8;
    A.nmat = nmat;
    for (int i = 0; i < 3; i++) {
        const DevWeight& wi = *ws[i < nmat ? i : 0];
        A.mat[i].W = wi.data;
        A.mat[i].wref = wi.wref;
        A.mat[i].bias = i < nmat ? bias[i] : nullptr;
        A.mat[i].y = i < nmat ? y[i] : nullptr;
        A.mat[i].N = (int)wi.n;
        A.mat[i].tile0 = 0;
    }
    if (w.dt == DT_Q4_K) return launch_dt<DT_Q4_K>(A, (int)rows, stream);
    if (w.dt == DT_Q6_K) return launch_dt<DT_Q6_K>(A, (int)rows, stream);
    return hipErrorInvalidValue;
}

}  // namespace mimg
