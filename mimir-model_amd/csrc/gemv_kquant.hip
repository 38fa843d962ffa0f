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
// lane are in flight (the GEMV is bound by HBM latency x bandwidth). The U
// pairs of a group are U rows of one block, so the group reads that block's
// activation quants once (through L1: they are shared by all rows), before
// its weight loads. For a pair, lane l of the group loads 16 bytes of the
// block's quants, forms its part of S with v_dot4_i32_i8, and the group sums
// the parts with three DPP steps (integer, so exact in any order). The exact
// (S, M) and the two f32 scale products of every pair go to LDS; then one
// lane per (row, activation row) runs the serial float chain over the blocks
// in order. (A tiled kernel walking each row's blocks in order, and a
// persistent software-pipelined variant, measured slower on MI355X at these
// shapes.)
//
// Rows of x the quantizer refused and rows of w with a non-finite block scale
// take the float32 path (reference linearA8, interp/fast.go:323-377), in the
// reference's AVX2 order (f32path.hpp).
#include <algorithm>
#include <climits>
#include <cstring>

#include "decoder_math.hpp"
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
    // swiglu in the epilogue (one row; mat[0] gate, mat[1] up): out[n] =
    // swiglu.v1 of (gate row n, up row n) with the reference's pieces
    float* sw;
    int64_t sw_total, sw_chunk;
};

template <uint32_t DT>
struct KQ {
    static constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    static constexpr int S16PB = DT == DT_Q4_K ? 8 : 16;  // s16 entries per block
};

// Pairs per group and iteration (all their weight loads in flight at once).
constexpr int PAIRS_U = 4;

// With U dividing R, the U-row quads (block b, rows r0..r0+U-1) of group g:
// the pair base pb = p0 + U*g (< npairs) names quad pb/U, block-fastest (b =
// (pb/U) % nb), so that the eight groups of a wave read eight consecutive
// blocks of the same rows (measured: Q6_K down 13.6 -> 12.9 us against
// block-major quads, gate unchanged).
template <int R, int U>
__device__ __forceinline__ void quad_of(int pb, int nb, int& b, int& r0) {
    const int q = pb / U;
    const int rq = q / nb;
    b = q - rq * nb;
    r0 = rq * U;
}

// Pairs are numbered block-major (p = b*R + r), and group g of an iteration
// takes pairs p0 + U*g + [0, U) (with U dividing R, the quad of quad_of
// instead; the table slots stay (r*nb + b)*M): with U dividing R these are U rows of one
// block, so the group's activation for the iteration is one block's. Its
// loads (for one activation row) and the row flags are issued before the
// weights: the load counter being in order, anything issued after the
// weights would wait for all of them. Every load is unconditional (clamped
// in bounds) in straight-line code, and every loaded pair is consumed.
// SW (swiglu epilogue, M = 1, R = 2U): local rows 0..U-1 are gate rows
// tile*U.., rows U..2U-1 the same rows of up; a quad of U rows is one
// matrix's, so each quad loads from its matrix's tile base. The rows'
// results meet in LDS and out[n] = swiglu(gate[n], up[n]) is written.
// One workgroup's tile `tile` of the matrix A.W (A.wref, A.bias, A.y, A.N
// and A.y_stride are that matrix's; SW reads gate and up from A.mat[0..1]).
template <uint32_t DT, int M, int R, bool SW, int U = PAIRS_U>
__device__ __forceinline__ void pairs_tile(GemvArgs A, int tile, uint8_t* smem) {
    constexpr bool SHARED = R % U == 0;  // a group's U pairs share one block
    constexpr bool PRE = M == 1;         // activation loaded before the weights
    static_assert(!SW || (M == 1 && R == 2 * U && SHARED), "swiglu epilogue: one row, a gate and an up quad");
    const int g = threadIdx.x >> 3, l = threadIdx.x & 7, t = threadIdx.x;
    const int nb = A.nb, row0 = tile * (SW ? U : R), npairs = R * nb;
    // The tile's R rows: a 4-byte-aligned base (Q6_K rows are 2-byte
    // aligned) and 32-bit offsets from it (SW: the U rows of each matrix).
    const int64_t tbyte = (int64_t)row0 * A.rb;
    const uint8_t* Wt = A.W + (tbyte & ~(int64_t)3);
    const uint32_t tadj = (uint32_t)(tbyte & 3), rb32 = (uint32_t)A.rb;
    const uint8_t* Wt1 = SW ? A.mat[1].W + (tbyte & ~(int64_t)3) : Wt;
    const int rlast = SW ? R - 1 : min(R, A.N - row0) - 1;  // last row of the tile in the matrix
    i32x4* part = (i32x4*)smem;                                 // [R][nb][M]: S, M term, bits(d*dx), bits(dmin*dx)
    int* refused = (int*)(smem + (size_t)R * nb * M * 16);      // [R*M]: the pair takes the float32 path

    // Lane t < R*M owns (weight row t/M, activation row t%M) at the end.
    // Every lane loads the flags and bias of a clamped (row, activation row)
    // first and looks at them last (a branch or a scalar load here would
    // wait for them before the weights are requested).
    int fm = min(t, R * M - 1) % M;
    asm volatile("v_mov_b32 %0, %1" : "=v"(fm) : "v"(fm));  // a vector index: ok[] through the vector cache
    const int fr = min(t, R * M - 1) / M;
    const PairMat& FM = SW && fr >= U ? A.mat[1] : A.mat[0];
    const int frow = SW ? row0 + (fr & (U - 1)) : min(row0 + fr, A.N - 1);
    const int wr = SW ? FM.wref[frow] : A.wref[frow], okm = A.ok[fm];
    const float* fbias = SW ? FM.bias : A.bias;
    const float bias = fbias ? fbias[frow] : 0.f;
    __builtin_amdgcn_sched_barrier(0);

    for (int p0 = 0; p0 < npairs; p0 += 32 * U) {
        ActLane pre[SHARED ? 1 : U];
        if constexpr (PRE) {
#pragma unroll
            for (int u = 0; u < (SHARED ? 1 : U); u++) {
                int pbk;
                if constexpr (SHARED) {
                    int r0;
                    quad_of<R, U>(min(p0 + U * g, npairs - U), nb, pbk, r0);
                } else {
                    pbk = min(p0 + U * g + u, npairs - 1) / R;
                }
                pre[u] = act_lane<DT>(A.q, A.s16, A.d32, A.K, 0, pbk, l);
            }
        }
        // Keep the issue order: activation, then all weights, then compute.
        __builtin_amdgcn_sched_barrier(0);
        u32x4 hdr[U], qv[U];
        Q6KRaw raw[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            int b, r;
            if constexpr (SHARED) {
                int r0;
                quad_of<R, U>(min(p0 + U * g, npairs - U), nb, b, r0);  // rows r0..r0+U-1 of block b
                r = min(r0 + u, rlast);
            } else {
                const int p = min(p0 + U * g + u, npairs - 1);
                b = p / R;
                r = min(p - b * R, rlast);
            }
            const uint8_t* Wb = SW && r >= U ? Wt1 : Wt;
            const uint32_t off = tadj + (uint32_t)(SW ? (r & (U - 1)) : r) * rb32 + (uint32_t)b * KQ<DT>::BYTES;
            if constexpr (DT == DT_Q4_K) {
                hdr[u] = *(const u32x4*)(Wb + off);
                qv[u] = *(const u32x4*)(Wb + (off + 16 * l + 16));
            } else {
                raw[u] = q6k_load_at(Wb, off, l);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // Table slots of the group's pairs: (r*nb + b)*M + m.
        int slot0 = 0, pb = 0;
        if constexpr (SHARED) {
            pb = p0 + U * g;
            int b, r0;
            quad_of<R, U>(min(pb, npairs - U), nb, b, r0);
            slot0 = (r0 * nb + b) * M;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            bool store;
            int slot;
            if constexpr (SHARED) {
                store = pb < npairs;  // all U pairs of the group, or none
                slot = slot0 + u * nb * M;
            } else {
                const int pu = p0 + U * g + u;
                store = pu < npairs;
                const int p = min(pu, npairs - 1);
                const int b = p / R, r = p - b * R;
                slot = (r * nb + b) * M;
            }
#pragma unroll
            for (int m = 0; m < M; m++) {
                // Without PRE the activation is read here, after the weights
                // (once per iteration and activation row when SHARED).
                ActLane a;
                if constexpr (PRE) {
                    a = pre[SHARED ? 0 : u];
                } else {
                    // (Written per pair: read once for all U pairs, the M
                    // rows' activations would all stay in registers.)
                    int bk;
                    if constexpr (SHARED) {
                        int r0;
                        quad_of<R, U>(min(p0 + U * g, npairs - U), nb, bk, r0);
                    } else {
                        bk = min(p0 + U * g + u, npairs - 1) / R;
                    }
                    a = act_lane<DT>(A.q, A.s16, A.d32, A.K, m, bk, l);
                }
                const i32x4 v = pair_part<DT>(hdr[u], qv[u], raw[u], a, l);
                if (l == 0 && store) part[slot + m] = v;
            }
        }
    }
    const int flag = (wr != 0) | (okm == 0);
    if (t < R * M) refused[t] = flag;
    __syncthreads();

    // The serial float chain, one lane per (weight row, activation row).
    float* yr = (float*)(refused + R * M);  // SW: [R] the rows' results
    if (t < R * M) {
        const int r = t / M, m = t - r * M, row = SW ? row0 + (r & (U - 1)) : row0 + r;
        if (row < A.N && !flag) {
            float tot = 0.f, off = 0.f;
            for (int b = 0; b < nb; b++) {
                const i32x4 v = part[(r * nb + b) * M + m];
                tot = __builtin_fmaf((float)v.x, __int_as_float(v.z), tot);
                if (DT == DT_Q4_K) off = __builtin_fmaf((float)v.y, __int_as_float(v.w), off);
            }
            float res = DT == DT_Q4_K ? tot - off : tot;
            if (fbias) res += bias;
            if (SW) yr[r] = res;
            else A.y[(int64_t)m * A.y_stride + row] = res;
        }
    }
    // The float32 path for refused pairs, one group of eight lanes per pair.
    for (int qq = g; qq < R * M; qq += 32) {
        const int r = qq / M, m = qq - r * M, row = SW ? row0 + (r & (U - 1)) : row0 + r;
        if (row < A.N && refused[qq]) {
            const PairMat& RM = SW && r >= U ? A.mat[1] : A.mat[0];
            const uint8_t* Wr = SW ? RM.W : A.W;
            const float* br = SW ? RM.bias : A.bias;
            float res = f32dot_g8<DT>(Wr + (int64_t)row * A.rb, A.x + (int64_t)m * A.K, A.K, A.fused != 0);
            if (br) res += br[row];
            if (l == 0) {
                if (SW) yr[r] = res;
                else A.y[(int64_t)m * A.y_stride + row] = res;
            }
        }
    }
    if constexpr (SW) {
        // swiglu.v1 of (gate, up) row n: the reference's SiluMulF32 on its pieces
        __syncthreads();
        const int n = row0 + t;
        if (t < U && n < A.N) A.sw[n] = swiglu_at(yr[t], yr[t + U], n, A.sw_total, A.sw_chunk);
    }
}

template <uint32_t DT, int M, int R, bool SW = false, int U = PAIRS_U>
__global__ __launch_bounds__(256) void gemv_a8k_pairs_kernel(GemvArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    // This workgroup's matrix of the launch.
    int mi = 0;
    if (!SW && A.nmat > 1 && (int)blockIdx.x >= A.mat[1].tile0) mi = 1;
    if (!SW && A.nmat > 2 && (int)blockIdx.x >= A.mat[2].tile0) mi = 2;
    const PairMat P = mi == 0 ? A.mat[0] : mi == 1 ? A.mat[1] : A.mat[2];
    A.W = P.W;
    A.wref = P.wref;
    A.bias = P.bias;
    A.y = P.y;
    A.N = P.N;
    A.y_stride = P.N;
    pairs_tile<DT, M, R, SW, U>(A, (int)blockIdx.x - P.tile0, smem);
}

// gate and up at one row with swiglu in the epilogue (Q4_K, N % U == 0).
static hipError_t launch_pairs_swiglu(GemvArgs A, hipStream_t stream) {
    constexpr int U = PAIRS_U, R = 2 * U;
    A.mat[0].tile0 = A.mat[1].tile0 = 0;
    const int tiles = A.N / U;
    const size_t lds = (size_t)R * A.nb * 16 + (size_t)R * 4 + (size_t)R * 4;
    hipLaunchKernelGGL((gemv_a8k_pairs_kernel<DT_Q4_K, 1, R, true>), dim3((unsigned)tiles), dim3(256), lds, stream, A);
    return hipGetLastError();
}

template <uint32_t DT, int M, int R, int U = PAIRS_U>
static hipError_t launch_pairs_r(GemvArgs A, hipStream_t stream) {
    int tiles = 0;
    for (int i = 0; i < A.nmat; i++) {
        A.mat[i].tile0 = tiles;
        tiles += (A.mat[i].N + R - 1) / R;
    }
    const size_t lds = (size_t)R * A.nb * M * 16 + (size_t)R * M * 4;
    hipLaunchKernelGGL((gemv_a8k_pairs_kernel<DT, M, R, false, U>), dim3((unsigned)tiles), dim3(256), lds, stream, A);
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

bool gemv_swiglu_ok(const DevWeight& gate, const DevWeight& up) {
    return gate.dt == DT_Q4_K && up.dt == DT_Q4_K && gate.n == up.n && gate.k == up.k && gate.k % 256 == 0 &&
           gate.n % PAIRS_U == 0 && gate.k <= 16384 && gate.n <= (1 << 30);
}

hipError_t launch_gemv_a8k_swiglu(const DevWeight& gate, const DevWeight& up, const ActPtrs& a, const float* x,
                                  const float* const* bias, float* out, int64_t total, int64_t chunk,
                                  hipStream_t stream) {
    if (!gemv_swiglu_ok(gate, up)) return hipErrorInvalidValue;
    GemvArgs A;
    A.W = gate.data;
    A.rb = gate.row_bytes;
    A.N = (int)gate.n;
    A.nb = (int)(gate.k / 256);
    A.K = gate.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.s16 = a.xs;
    A.ok = a.ok;
    A.wref = gate.wref;
    A.x = x;
    A.bias = bias ? bias[0] : nullptr;
    A.y = nullptr;
    A.y_stride = gate.n;
    A.fused = 1;
    A.nmat = 2;
    const DevWeight* w2[2] = {&gate, &up};
    for (int i = 0; i < 3; i++) {
        const DevWeight& wi = *w2[i < 2 ? i : 0];
        A.mat[i].W = wi.data;
        A.mat[i].wref = wi.wref;
        A.mat[i].bias = i < 2 && bias ? bias[i] : nullptr;
        A.mat[i].y = nullptr;
        A.mat[i].N = (int)wi.n;
        A.mat[i].tile0 = 0;
    }
    A.sw = out;
    A.sw_total = total;
    A.sw_chunk = chunk;
    return launch_pairs_swiglu(A, stream);
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
    A.sw = nullptr;
    A.sw_total = A.sw_chunk = 0;
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

// Independent one-row products in one launch (mimg_linear_a8_set_dev): the
// segments are matrices with activation rows of their own (a decoder
// layer's linear set with an input per matrix), Q4_K and Q6_K mixed, K per
// segment. A workgroup finds its segment in the argument table through the
// argument segment pointer (indexing the by-value table with the
// workgroup's segment would make the compiler copy it to private memory)
// and runs that matrix's tile exactly as the pairs kernel does, so every
// output is bit for bit the separate call's.
template <int R4, int R6, int U6>
__global__ __launch_bounds__(256) void gemv_a8k_set_kernel(SetArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    const SetArgs* S = (const SetArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    const int bid = (int)blockIdx.x;
    // the first workgroups of the segments in one 64-byte scalar load
    // (unused entries hold INT_MAX)
    int si = 0;
#pragma unroll
    for (int i = 1; i < SET_MAXSEG; i++) si += bid >= S->tile0[i] ? 1 : 0;
    const SetSeg* s = &S->seg[si];
    GemvArgs A;
    A.W = s->W;
    A.rb = s->rb;
    A.N = s->N;
    A.nb = s->nb;
    A.K = s->K;
    A.q = s->q;
    A.d32 = s->d32;
    A.s16 = s->s16;
    A.ok = s->ok;
    A.wref = s->wref;
    A.x = s->x;
    A.bias = s->bias;
    A.y = s->y;
    A.y_stride = s->N;
    A.fused = 1;
    A.nmat = 1;
    A.sw = nullptr;
    A.sw_total = A.sw_chunk = 0;
    const int tile = bid - S->tile0[si];
    if (s->dt == DT_Q4_K) pairs_tile<DT_Q4_K, 1, R4, false>(A, tile, smem);
    else pairs_tile<DT_Q6_K, 1, R6, false, U6>(A, tile, smem);
}

// Rows per workgroup in a set launch (the launch has thousands of tiles, so
// the standalone launch's rule of at least 1024 workgroups does not apply).
// One launch for both dtypes measured faster than a launch per dtype
// (cfg1 set 39.0 against 41.0 us a step).
constexpr int SET_R4 = 8, SET_R6 = 8;
// Q6_K pairs in flight per group of eight lanes: two keep the launch at 64
// VGPRs (eight waves a SIMD for the Q4_K tiles too; measured on MI355X, the
// cfg1 set 34.3 -> 32.0 us with eight Q6_K rows a workgroup instead of four).
constexpr int SET_U6 = 2;

static int set_rows(uint32_t dt) { return dt == DT_Q4_K ? SET_R4 : SET_R6; }

// Segments in launch order, the longest workgroups first (weight bytes a
// workgroup reads), so that the grid's tail is made of short ones; tile0 of
// each set here.
static hipError_t launch_set(const SetArgs& in, hipStream_t stream) {
    SetArgs a;
    memset(&a, 0, sizeof a);
    for (int i = 0; i < in.nseg; i++) a.seg[a.nseg++] = in.seg[i];
    if (a.nseg == 0) return hipSuccess;
    auto wg_bytes = [](const SetSeg& s) {
        return (int64_t)set_rows((uint32_t)s.dt) * s.nb * (s.dt == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES);
    };
    std::stable_sort(a.seg, a.seg + a.nseg,
                     [&](const SetSeg& x, const SetSeg& y) { return wg_bytes(x) > wg_bytes(y); });
    int tiles = 0, nbmax = 1;
    for (int i = 0; i < SET_MAXSEG; i++) a.tile0[i] = INT_MAX;
    for (int i = 0; i < a.nseg; i++) {
        const int R = set_rows((uint32_t)a.seg[i].dt);
        a.tile0[i] = tiles;
        tiles += (a.seg[i].N + R - 1) / R;
        nbmax = a.seg[i].nb * R > nbmax ? a.seg[i].nb * R : nbmax;
    }
    const int rmax = SET_R4 > SET_R6 ? SET_R4 : SET_R6;
    const size_t lds = (size_t)nbmax * 16 + (size_t)rmax * 4;
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_a8k_set_kernel<SET_R4, SET_R6, SET_U6>), dim3((unsigned)tiles), dim3(256), lds, stream, a);
    return hipGetLastError();
}

hipError_t launch_gemv_a8k_set(const SetArgs& a, hipStream_t stream) {
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].dt != (int32_t)DT_Q4_K && a.seg[i].dt != (int32_t)DT_Q6_K) return hipErrorInvalidValue;
    return launch_set(a, stream);
}

}  // namespace mimg
