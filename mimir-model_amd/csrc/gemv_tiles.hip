// Decode GEMV for one activation row, tile-looping form: Q4_K / Q6_K
// weights x 8-bit activations in blocks of 256 (dequant_matmul_a8.v2,
// block = 256), the numerics of gemv_kquant.hip bit for bit (reference
// dotQ8KRef, internal/kernels/q8k_test.go:38-102).
//
// A grid of a few workgroups per CU walks the row tiles (R rows each) of up
// to three matrices that share the activations. Per tile, a workgroup
//   1. loads the refusal flags and biases of the tile's rows (lanes t < R),
//   2. issues the weight loads of its (row, block) pairs, U per group of
//      eight lanes,
//   3. while those are in flight, runs the serial float chain of the
//      previous tile (lanes t < R) from the other half of a double-buffered
//      pair table in LDS,
//   4. forms the exact int32 block sums of the tile's pairs into the current
//      half, then meets the others at one barrier.
// The activation row (quants, block sums, scales) is copied into LDS once
// per workgroup with global_load_lds, so the compute phase reads no global
// memory: a global read issued after the weight loads would wait for all of
// them, the load counter being in order. Compared with one workgroup per
// tile, fewer loads are in flight at once and they return roughly in issue
// order, so compute spreads over the kernel instead of piling up at its end.
//
// Rows of W with a non-finite block scale, and a refused activation row,
// take the float32 path (reference interp/fast.go:323-377) after the walk.
#include "f32path.hpp"
#include "kquant_lane.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

struct TileMat {
    const uint8_t* W;
    const uint8_t* wref;
    const float* bias;
    float* y;
    int N;
    int tile0;  // first tile of this matrix
};

struct TilesArgs {
    TileMat mat[3];
    int nmat;
    int ntiles;
    int64_t rb;          // bytes per weight row
    int nb;              // blocks of 256 per row
    int64_t K;
    const int8_t* q;     // the activation row: q [K]
    const float* d32;    // [K/32]
    const int16_t* s16;  // Q4_K: xs [K/32]; Q6_K: ys16 [K/16]
    const int32_t* ok;   // [1]
    const float* x;      // f32 activations (fallback)
    int fused;           // float32 fallback order (rows of the whole call <= 8)
};

constexpr int TILES_MAXK = 16384;

// The matrix a tile belongs to (selected without indexing the argument
// array, which would go through scratch memory).
__device__ __forceinline__ TileMat tile_mat(const TilesArgs& A, int tile) {
    const bool m2 = A.nmat > 2 && tile >= A.mat[2].tile0;
    const bool m1 = A.nmat > 1 && tile >= A.mat[1].tile0;
    return m2 ? A.mat[2] : m1 ? A.mat[1] : A.mat[0];
}

template <uint32_t DT, int R>
__global__ __launch_bounds__(256) void gemv_a8k_tiles_kernel(TilesArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int U = 4;
    constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    constexpr int S16PB = DT == DT_Q4_K ? 8 : 16;
    const int t = threadIdx.x, g = t >> 3, l = t & 7;
    const int nb = A.nb, np = R * nb;
    const int64_t K = A.K;

    // LDS: pair tables [2][R*nb] (S, M term, bits(d*dx), bits(dmin*dx)),
    // then the staged row q [K], s16 [nb*S16PB], dx [nb], and a flag.
    i32x4* part0 = (i32x4*)smem;
    int8_t* sq = (int8_t*)(smem + 2 * (size_t)np * 16);
    int16_t* ss = (int16_t*)(sq + K);
    float* sdx = (float*)(ss + nb * S16PB);
    int* any_ref = (int*)(sdx + nb);

    {
        const int wave = t >> 6, nq = (int)(K / 16), ns = nb * S16PB / 8;
#pragma unroll
        for (int j = 0; j < TILES_MAXK / 16 / 256; j++)
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
    if (t == 0) *any_ref = 0;
    const int ok0 = A.ok[0];

    // The float chain of tile `tile` (lanes t < R) from pair table pp.
    auto chain = [&](int tile, const i32x4* pp, int ref, float bias) {
        const TileMat P = tile_mat(A, tile);
        const int row = (tile - P.tile0) * R + t;
        if (t < R && row < P.N) {
            if (ref) {
                *any_ref = 1;
            } else {
                const i32x4* pr = pp + t * nb;
                float tot = 0.f, off = 0.f;
                for (int b = 0; b < nb; b++) {
                    const i32x4 v = pr[b];
                    tot = __builtin_fmaf((float)v.x, __int_as_float(v.z), tot);
                    if (DT == DT_Q4_K) off = __builtin_fmaf((float)v.y, __int_as_float(v.w), off);
                }
                float res = DT == DT_Q4_K ? tot - off : tot;
                if (P.bias) res += bias;
                P.y[row] = res;
            }
        }
    };

    int prev = -1, p_ref = 0, buf = 0;
    float p_bias = 0.f;
    bool first = true;
    for (int tile = blockIdx.x; tile < A.ntiles; tile += gridDim.x) {
        const TileMat P = tile_mat(A, tile);
        const int row0 = (tile - P.tile0) * R;
        int c_ref = 0;
        float c_bias = 0.f;
        if (t < R && row0 + t < P.N) {
            c_ref = (P.wref[row0 + t] != 0) | (ok0 == 0);
            if (P.bias) c_bias = P.bias[row0 + t];
        }
        i32x4* part = part0 + buf * np;
        for (int p0 = 0; p0 < np; p0 += 32 * U) {
            u32x4 hdr[U], qv[U];
            Q6KRaw raw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + g + 32 * u;
                if (p < np) {
                    const int r = p / nb, b = p - r * nb;
                    const int row = min(row0 + r, P.N - 1);
                    const uint8_t* blk = P.W + (int64_t)row * A.rb + (int64_t)b * BYTES;
                    if constexpr (DT == DT_Q4_K) {
                        hdr[u] = *(const u32x4*)blk;
                        qv[u] = *(const u32x4*)(blk + 16 + 16 * l);
                    } else {
                        raw[u] = q6k_load(blk, l);
                    }
                }
            }
            if (p0 == 0) {
                if (prev >= 0) chain(prev, part0 + (buf ^ 1) * np, p_ref, p_bias);
                if (first) {
                    // The staged row (and this wave's first weights) have landed.
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    first = false;
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = p0 + g + 32 * u;
                if (p >= np) break;  // uniform within the group
                const int r = p / nb, b = p - r * nb;
                i32x4 v;
                if constexpr (DT == DT_Q4_K) {
                    const Q4KLane w = q4k_lane(hdr[u], qv[u], l);
                    const int8_t* yb = sq + 256 * b + w.yoff;
                    v.x = group8_sum(q4k_part(w, *(const u32x4*)yb, *(const u32x4*)(yb + 32)));
                    v.y = group8_sum(w.mm * (int)ss[8 * b + l]);
                    const float dx = sdx[b];
                    v.z = __float_as_int(w.d * dx);
                    v.w = __float_as_int(w.dmin * dx);
                } else {
                    const Q6KLane w = q6k_lane(raw[u], l);
                    const int8_t* yb = sq + 256 * b;
                    v.x = group8_sum(q6k_part(w, *(const u32x4*)(yb + w.eL), *(const u32x4*)(yb + w.eL + 64),
                                              ss[16 * b + (w.eL >> 4)], ss[16 * b + ((w.eL + 64) >> 4)]));
                    v.y = 0;
                    v.z = __float_as_int(w.d * sdx[b]);
                    v.w = 0;
                }
                if (l == 0) part[r * nb + b] = v;
            }
        }
        __syncthreads();
        prev = tile;
        p_ref = c_ref;
        p_bias = c_bias;
        buf ^= 1;
    }
    if (prev >= 0) chain(prev, part0 + (buf ^ 1) * np, p_ref, p_bias);

    // Refused rows of this workgroup's tiles: the float32 path, one group of
    // eight lanes per row.
    __syncthreads();
    if (*any_ref == 0) return;
    for (int tile = blockIdx.x; tile < A.ntiles; tile += gridDim.x) {
        const TileMat P = tile_mat(A, tile);
        for (int r = g; r < R; r += 32) {
            const int row = (tile - P.tile0) * R + r;
            if (row < P.N && (P.wref[row] != 0 || ok0 == 0)) {
                float res = f32dot_g8<DT>(P.W + (int64_t)row * A.rb, A.x, K, A.fused != 0);
                if (P.bias) res += P.bias[row];
                if (l == 0) P.y[row] = res;
            }
        }
    }
}

static size_t tiles_lds(int R, int nb, int64_t K, int s16pb) {
    return 2 * (size_t)R * nb * 16 + (size_t)K + (size_t)nb * s16pb * 2 + (size_t)nb * 4 + 16;
}

template <uint32_t DT, int R>
static hipError_t launch_tiles_r(TilesArgs A, int wgs_per_cu, hipStream_t stream) {
    int tiles = 0;
    for (int i = 0; i < A.nmat; i++) {
        A.mat[i].tile0 = tiles;
        tiles += (A.mat[i].N + R - 1) / R;
    }
    A.ntiles = tiles;
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    const int grid = tiles < cus * wgs_per_cu ? tiles : cus * wgs_per_cu;
    const size_t lds = tiles_lds(R, A.nb, A.K, DT == DT_Q4_K ? 8 : 16);
    hipLaunchKernelGGL((gemv_a8k_tiles_kernel<DT, R>), dim3((unsigned)grid), dim3(256), lds, stream, A);
    return hipGetLastError();
}

bool gemv_tiles_ok(const DevWeight& w, int64_t rows) {
    return rows == 1 && (w.dt == DT_Q4_K || w.dt == DT_Q6_K) && w.k % 256 == 0 && w.k <= TILES_MAXK;
}

hipError_t launch_gemv_a8k_tiles(const DevWeight* const* ws, int nmat, const ActPtrs& a, int64_t total_rows,
                                 const float* x, const float* const* bias, float* const* y, int wgs_per_cu,
                                 hipStream_t stream) {
    if (nmat < 1 || nmat > 3 || wgs_per_cu < 1) return hipErrorInvalidValue;
    const DevWeight& w = *ws[0];
    if (!gemv_tiles_ok(w, 1)) return hipErrorInvalidValue;
    for (int i = 0; i < nmat; i++)
        if (ws[i]->dt != w.dt || ws[i]->k != w.k || ws[i]->n <= 0) return hipErrorInvalidValue;
    TilesArgs A;
    A.nmat = nmat;
    A.rb = w.row_bytes;
    A.nb = (int)(w.k / 256);
    A.K = w.k;
    A.q = a.q;
    A.d32 = a.d32;
    A.s16 = w.dt == DT_Q4_K ? a.xs : a.ys16;
    A.ok = a.ok;
    A.x = x;
    A.fused = total_rows <= 8;
    for (int i = 0; i < 3; i++) {
        const DevWeight& wi = *ws[i < nmat ? i : 0];
        A.mat[i].W = wi.data;
        A.mat[i].wref = wi.wref;
        A.mat[i].bias = i < nmat ? bias[i] : nullptr;
        A.mat[i].y = i < nmat ? y[i] : nullptr;
        A.mat[i].N = (int)wi.n;
        A.mat[i].tile0 = 0;
    }
    // Rows per tile: one batch of U pairs per group of eight lanes.
    const int nb = A.nb;
    if (w.dt == DT_Q4_K) {
        if (8 * nb <= 128) return launch_tiles_r<DT_Q4_K, 8>(A, wgs_per_cu, stream);
        if (4 * nb <= 128) return launch_tiles_r<DT_Q4_K, 4>(A, wgs_per_cu, stream);
        if (2 * nb <= 128) return launch_tiles_r<DT_Q4_K, 2>(A, wgs_per_cu, stream);
        return launch_tiles_r<DT_Q4_K, 1>(A, wgs_per_cu, stream);
    }
    if (8 * nb <= 128) return launch_tiles_r<DT_Q6_K, 8>(A, wgs_per_cu, stream);
    if (4 * nb <= 128) return launch_tiles_r<DT_Q6_K, 4>(A, wgs_per_cu, stream);
    if (2 * nb <= 128) return launch_tiles_r<DT_Q6_K, 2>(A, wgs_per_cu, stream);
    return launch_tiles_r<DT_Q6_K, 1>(A, wgs_per_cu, stream);
}

}  // namespace mimg
