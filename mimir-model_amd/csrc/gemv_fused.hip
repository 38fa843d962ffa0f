// Decode GEMV for one activation row with the 8-bit quantization fused in:
// dequant_matmul_a8.v2, block = 256, M = 1, Q4_K and Q6_K weights, for up
// to three weight matrices that share the activation row (q, k, v of a
// decoder layer; gate and up) in one launch.
//
// Each 256-thread workgroup owns R rows of one matrix. It first issues the
// loads of x, of its rows' flags and of the weights of its (row, block)
// pairs, then quantizes x into LDS while they are in flight (every
// workgroup quantizes the same row the same way, so no second launch and no
// global workspace), then forms the exact int32 block sums of its pairs (as
// gemv_kquant.hip, block-major pairs) and runs the serial float chain of
// each row in block order. Where the tiles fill every CU two or three times
// over, a workgroup holds two or three such 256-thread teams, each with its
// own tile, and only the first quantizes x into the LDS row they share: the
// row's re-reads per CU drop by that factor (measured on MI355X: the cfg1
// layer set 52.7 -> 50.6 us per step, q/k/v 768 tiles as 256 workgroups of
// three teams, o 512 tiles as 256 of two).
//
// Quantization (reference Q8.QuantizeBlocks, internal/kernels/q8.go:50-97):
// per block of 256, amax = max|x| (the row is refused if any |x| is NaN or
// above 2^60); q = RoundToEven(127 x / amax) of the exact quotient
// (quant_rne.hpp); d = amax/127 (correctly rounded f32 division); per-16 and
// per-32 sums of q.
#include "decoder_math.hpp"
#include "f32path.hpp"
#include "kquant_lane.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

constexpr int DPP_ROW_ROR1 = 0x121, DPP_ROW_ROR2 = 0x122, DPP_ROW_ROR4 = 0x124, DPP_ROW_ROR8 = 0x128;

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR8, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR4, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR2, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR1, 0xF, 0xF, false)));
    return v;
}

struct QuantLds {
    int8_t* q;       // [K]
    float* dx;       // [nb]
    int16_t* xs;     // [K/32]
    int16_t* ys16;   // [K/16]
};

// Quantizes block b of the row into LDS from this thread's 16 values (16
// threads, one DPP row, per block of 256; thread j of the row holds
// elements 16j..16j+15). Returns this thread's refusal flag.
__device__ __forceinline__ bool quantize_block_lds(const float4 (&v)[4], int b, int j, const QuantLds& Q) {
    const float xv[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                          v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
    float m = 0.f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = fabsf(xv[i]);
        bad |= !(a <= 0x1p60f);
        m = fmaxf(m, a);
    }
    const float amax = row16_max(m);
    const bool quant = amax > 0.f && amax <= 0x1p60f;
    const float inv = quant ? 1.0f / amax : 0.f;
    // the fast rounding for all 16 (branch-free), the exact one where it
    // cannot decide (about one element in 2^11)
    int qs[16];
    bool fast[16];
#pragma unroll
    for (int i = 0; i < 16; i++) fast[i] = quant_rne_fast(xv[i], amax, inv, qs[i]);
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (quant && !fast[i]) qs[i] = quant_rne(xv[i], amax, inv);
    uint32_t w[4] = {0, 0, 0, 0};
    int s16 = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int q = quant ? qs[i] : 0;
        s16 += q;
        w[i >> 2] |= (uint32_t)(q & 0xFF) << (8 * (i & 3));
    }
    *(u32x4*)(Q.q + 256 * b + 16 * j) = u32x4{w[0], w[1], w[2], w[3]};
    const int s32 = s16 + __builtin_amdgcn_mov_dpp(s16, DPP_QUAD_1032, 0xF, 0xF, false);
    Q.ys16[16 * b + j] = (int16_t)s16;
    if ((j & 1) == 0) Q.xs[8 * b + (j >> 1)] = (int16_t)s32;
    if (j == 0) Q.dx[b] = amax / 127.0f;
    return bad;
}

__device__ __forceinline__ void load_x16(const float* __restrict__ x, int b, int j, float4 (&v)[4]) {
    const float4* xp = (const float4*)(x + 256 * b + 16 * j);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = xp[i];
}

struct FusedMat {
    const uint8_t* W;
    const uint8_t* wref;
    const float* bias;
    float* y;
    int64_t rb;
    int N;
    uint32_t dt;
    int R;       // rows per workgroup
    int tile0;   // first workgroup of this matrix
};

struct FusedArgs {
    FusedMat mat[3];
    int nmat;
    const float* x;
    int64_t K;
    int nb;
    // rms_norm in front (NORM kernels): y = rms_norm(x + resid) * scale is
    // quantized; x + resid goes to x_out (tile 0 of matrix 0 writes it)
    const float* resid;
    const float* scale;
    float eps;
    float* x_out;
    // rope.v1 and the cache scatter in the epilogue (matrices q, k, v of a
    // decoder layer at one row; rope_kv_kernel's pairs and steps): rows of q
    // and k are dealt to workgroups in rotation pairs, so that a workgroup
    // holds both rows of each pair it rotates
    int rope;
    const int64_t* pos;   // [1]
    const int64_t* cidx;  // [1]
    const double* inv_freq;
    int D, rotary, interleaved, f16;
    int64_t C;
    void* kc;
    void* vc;
    // LDS: the quantized row (and the normed row) shared by the workgroup's
    // teams, then one region per team (pair table, flags, rope values)
    int lds_row, lds_team;
};

// Row of local row r of tile `tile` of matrix mi: with rope (RD = the head
// dim, 64 or 128; 0 without), q (mi 0) and k (mi 1) rows come in pairs:
// local rows 2j, 2j+1 are rope_kv_kernel's dims (a, b) of pair
// P = tile*R/2 + j (head P / (RD/2), pair P % (RD/2)); v and every matrix
// without rope keep their rows in order.
template <int RD>
__device__ __forceinline__ int fused_row(const FusedArgs& A, int mi, int tile, int R, int r) {
    if (RD == 0 || mi == 2) return tile * R + r;
    constexpr int half = RD / 2;
    const int h2 = A.rotary / 2;
    const int P = tile * (R / 2) + (r >> 1), hh = P / half, i = P - hh * half;
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

// rms_norm.v1 of the row (rms_norm_kernel's order: thread t sums the float4s
// t + 256k of x + resid, then the wave and workgroup sums), and the
// quantization of y straight from that layout: float4 t + 256k is lane t%64
// of chunk 4k + t/64, one block of 256 per wave (quantize_act.hip's
// layout). y also goes to LDS (yl) for the float32 path of refused rows.
// Returns this thread's refusal flag. K % 1024 == 0, K <= 4096.
constexpr int NORM_R = 4;  // float4s per thread of the normed row, K <= 4096
// Rounds of the normed row's quantization the lead team runs (the rest go
// to the other teams, NORM_PER each).
template <int TEAMS>
constexpr int NORM_KL = TEAMS == 1 ? NORM_R : 2;
template <int TEAMS>
constexpr int NORM_PER = TEAMS == 1 ? 0 : (NORM_R - 2) / (TEAMS - 1);

// The row's loads, issued before the weights (the load counter retires in
// order): x, resid, scale as float4s t + 256k (clamped; used where inside).
struct NormRegs {
    float4 x[NORM_R], r[NORM_R], s[NORM_R];
};
// (The lead team loads x and resid of every round and the scale of the
// rounds it quantizes itself, KL; a helper team the scale of its rounds.)
template <int KL>
__device__ __forceinline__ void norm_load(const FusedArgs& A, NormRegs& N) {
    const int n4 = (int)(A.K / 4);
#pragma unroll
    for (int k = 0; k < NORM_R; k++) {
        const int i = min((int)threadIdx.x + 256 * k, n4 - 1);
        N.x[k] = ((const float4*)A.x)[i];
        if (A.resid) N.r[k] = ((const float4*)A.resid)[i];
        if (k < KL && A.scale) N.s[k] = ((const float4*)A.scale)[i];
    }
}
template <int PER>
__device__ __forceinline__ void norm_load_helper(const FusedArgs& A, NormRegs& N, int k0) {
    const int n4 = (int)(A.K / 4), t = threadIdx.x & 255;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = min(t + 256 * (k0 + j), n4 - 1);
        if (A.scale) N.s[j] = ((const float4*)A.scale)[i];
    }
}

// One round k of the normed row (float4 t + 256k of it, t the thread of its
// team): y = (v*inv)*scale to yl, quantized into Q as block (t + 256k)/64.
// Returns the lane's refusal flag.
__device__ __forceinline__ bool norm_round(const FusedArgs& A, int t, int k, float4 v, float4 s4, float inv, float* yl,
                                           const QuantLds& Q) {
    const int lane = t & 63, i = t + 256 * k;
    float4 o = {v.x * inv, v.y * inv, v.z * inv, v.w * inv};
    if (A.scale) {
        o.x = o.x * s4.x;
        o.y = o.y * s4.y;
        o.z = o.z * s4.z;
        o.w = o.w * s4.w;
    }
    ((float4*)yl)[i] = o;
    // block b = i / 64 of 256: this wave's, lane's four at 4*lane
    const int b = i >> 6;
    const float xv[4] = {o.x, o.y, o.z, o.w};
    float av[4] = {fabsf(o.x), fabsf(o.y), fabsf(o.z), fabsf(o.w)};
    bool lbad = false;
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        lbad |= !(av[e] <= 0x1p60f);
        m = fmaxf(m, av[e]);
    }
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_QUAD_1032, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_QUAD_2301, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_HALF_MIRROR, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), DPP_ROW_MIRROR, 0xF, 0xF, false)));
    m = fmaxf(m, lane_xor_f32<16>(m));
    m = fmaxf(m, lane_xor_f32<32>(m));
    const float amax = m;
    const bool bbad = __any(lbad);
    const bool quant = !bbad && amax > 0.f;
    const float qinv = quant ? 1.0f / amax : 0.f;
    int qv[4];
    bool fast[4];
#pragma unroll
    for (int e = 0; e < 4; e++) fast[e] = quant_rne_fast(xv[e], amax, qinv, qv[e]);
#pragma unroll
    for (int e = 0; e < 4; e++) qv[e] = !quant ? 0 : fast[e] ? qv[e] : quant_rne(xv[e], amax, qinv);
    *(uint32_t*)(Q.q + 4 * i) = (uint32_t)(qv[0] & 0xFF) | ((uint32_t)(qv[1] & 0xFF) << 8) |
                                ((uint32_t)(qv[2] & 0xFF) << 16) | ((uint32_t)(qv[3] & 0xFF) << 24);
    const int s4i = qv[0] + qv[1] + qv[2] + qv[3];
    int s16 = s4i + __builtin_amdgcn_mov_dpp(s4i, DPP_QUAD_1032, 0xF, 0xF, false);
    s16 += __builtin_amdgcn_mov_dpp(s16, DPP_QUAD_2301, 0xF, 0xF, false);
    const int s32 = s16 + __builtin_amdgcn_mov_dpp(s16, DPP_HALF_MIRROR, 0xF, 0xF, false);
    if ((lane & 3) == 0) Q.ys16[i >> 2] = (int16_t)s16;
    if ((lane & 7) == 0) Q.xs[i >> 3] = (int16_t)s32;
    if (lane == 0) Q.dx[b] = amax / 127.0f;
    return lbad;
}

__device__ __forceinline__ float norm_inv(const FusedArgs& A, const double* part) {
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    return (float)(1.0 / sqrt((double)(float)(tot / (double)A.K) + (double)A.eps));
}

// The lead team: x + resid of every round, the sum of squares, then the
// rounds k < KL; rounds from KL on go to the helper teams, which read
// x + resid from yl (written here before the barrier) and overwrite it with y.
template <int KL>
__device__ __forceinline__ bool norm_quantize_lds(const FusedArgs& A, const NormRegs& N, bool write_x, float* yl,
                                                  double* part, const QuantLds& Q) {
    constexpr int NR = NORM_R;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int n4 = (int)(A.K / 4);
    float4 v[NR];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < NR; k++) {
        const int i = t + 256 * k;
        v[k] = N.x[k];
        if (i < n4) {
            if (A.resid) {
                v[k].x = v[k].x + N.r[k].x;
                v[k].y = v[k].y + N.r[k].y;
                v[k].z = v[k].z + N.r[k].z;
                v[k].w = v[k].w + N.r[k].w;
            }
            if (write_x) ((float4*)A.x_out)[i] = v[k];
            if (k >= KL) ((float4*)yl)[i] = v[k];
            ss += (double)v[k].x * (double)v[k].x + (double)v[k].y * (double)v[k].y +
                  (double)v[k].z * (double)v[k].z + (double)v[k].w * (double)v[k].w;
        }
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) part[w] = ss;
    lds_barrier();
    const float inv = norm_inv(A, part);
    bool bad = false;
#pragma unroll
    for (int k = 0; k < KL; k++) {
        if (t + 256 * k >= n4) continue;  // uniform within the wave (K % 1024 == 0)
        bad |= norm_round(A, t, k, v[k], N.s[k], inv, yl, Q);
    }
    return bad;
}

// A helper team's rounds k0 .. k0 + PER - 1, after the lead's barrier.
template <int PER>
__device__ __forceinline__ bool norm_quantize_helper(const FusedArgs& A, const NormRegs& N, int k0, float* yl,
                                                     double* part, const QuantLds& Q) {
    const int t = threadIdx.x & 255, n4 = (int)(A.K / 4);
    lds_barrier();
    const float inv = norm_inv(A, part);
    bool bad = false;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int k = k0 + j;
        if (t + 256 * k >= n4) continue;  // uniform
        bad |= norm_round(A, t, k, ((const float4*)yl)[t + 256 * k], N.s[j], inv, yl, Q);
    }
    return bad;
}

template <uint32_t DT>
struct FusedRaw;
template <>
struct FusedRaw<DT_Q4_K> {
    u32x4 hdr, qv;
};
template <>
struct FusedRaw<DT_Q6_K> {
    Q6KRaw raw;
};

// A group's activation for block b, from the row quantized into LDS.
template <uint32_t DT>
__device__ __forceinline__ ActLane act_lane_lds(const QuantLds& Q, int b, int l) {
    ActLane a;
    const int8_t* yb = Q.q + 256 * b;
    if constexpr (DT == DT_Q4_K) {
        const int yoff = 64 * (l >> 1) + 16 * (l & 1);
        a.ya = *(const u32x4*)(yb + yoff);
        a.yh = *(const u32x4*)(yb + yoff + 32);
        a.sa = Q.xs[8 * b + l];
        a.sb = 0;
    } else {
        const int eL = 128 * (l >> 2) + 32 * ((l & 3) >> 1) + 16 * (l & 1);
        a.ya = *(const u32x4*)(yb + eL);
        a.yh = *(const u32x4*)(yb + eL + 64);
        a.sa = Q.ys16[16 * b + (eL >> 4)];
        a.sb = Q.ys16[16 * b + ((eL + 64) >> 4)];
    }
    a.dx = Q.dx[b];
    return a;
}

// The pairs are numbered block-major (p = b*R + r) and group g of an
// iteration takes pairs p0 + U*g + [0, U); with U dividing R (SHARED) these
// are U rows of one block, whose activation is read from LDS once. Weights
// are addressed as 32-bit offsets from the tile's base; the row flags and
// bias are loaded first and looked at last.
//
// A workgroup of several teams (256 threads each, one tile each) quantizes
// the row once: the lead team (threads 0..255) loads x and fills the shared
// LDS row while every team's weights are in flight; the other teams meet it
// at the same barriers. `smem` is the shared row, `tmem` the team's region.
template <uint32_t DT, int U, bool SHARED, bool NORM, int RD, int TEAMS>
__device__ __forceinline__ void fused_body(const FusedArgs& A, const FusedMat& F, int mi, int tile, uint8_t* smem,
                                           uint8_t* tmem, double* npart, int* wflag, int team) {
    const bool lead = team == 0;
    constexpr int nwaves = 4 * TEAMS;
    constexpr bool ROPE = RD != 0;
    constexpr int BYTES = DT == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const int nb = A.nb, R = F.R, np = R * nb;
    const int64_t K = A.K;
    const int t = threadIdx.x & 255, g = t >> 3, l = t & 7;
    const int row0 = tile * R;
    QuantLds Q;
    Q.q = (int8_t*)smem;
    Q.dx = (float*)(smem + K);
    Q.xs = (int16_t*)(Q.dx + nb);
    Q.ys16 = (int16_t*)(Q.xs + K / 32);
    float* yl = (float*)(smem + ((K + nb * 4 + (K / 32) * 2 + (K / 16) * 2 + 15) & ~(int64_t)15));  // NORM: [K] y
    i32x4* part = (i32x4*)tmem;
    int* refl = (int*)(part + (size_t)R * nb);  // [R]: the row's weight is refused
    float* yr = (float*)(tmem + (((size_t)((uint8_t*)(refl + R) - tmem) + 15) & ~(size_t)15));  // rope: [R]
    // rows as 32-bit offsets from the tile's first row (its lowest)
    const int rbase = fused_row<RD>(A, mi, tile, R, 0);
    const int64_t tbyte = (int64_t)rbase * F.rb;
    const uint8_t* Wt = F.W + (tbyte & ~(int64_t)3);
    const uint32_t tadj = (uint32_t)(tbyte & 3), rb32 = (uint32_t)F.rb;
    const int rlast = min(R, F.N - row0) - 1;

    // 1. x (the first 16 blocks; lead team), the row flags and bias, then
    // the first U pairs' weights, all in flight; the load counter retires in
    // order, so the quantizer waits for x alone.
    const int j = t & 15, bq = t >> 4;
    float4 xv[4];
    NormRegs N;
    if (lead) {
        if constexpr (NORM) norm_load<NORM_KL<TEAMS>>(A, N);
        else load_x16(A.x, min(bq, nb - 1), j, xv);
    } else if constexpr (NORM && TEAMS > 1) {
        norm_load_helper<NORM_PER<TEAMS>>(A, N, NORM_KL<TEAMS> + (team - 1) * NORM_PER<TEAMS>);
    }
    const int frow = min(fused_row<RD>(A, mi, tile, R, min(t, R - 1)), F.N - 1);
    const int wr = F.wref[frow];
    const float bias = F.bias ? F.bias[frow] : 0.f;
    const int64_t pidx = ROPE ? A.cidx[0] : 0;  // (the rope epilogue's cache index)
    // (rope: the position and this thread's pair frequency, before the weights)
    int rot_i = 0;
    if (ROPE) {
        const int P = tile * (R / 2) + min(t, R / 2 - 1);
        rot_i = P - (P / (RD / 2 > 0 ? RD / 2 : 1)) * (RD / 2 > 0 ? RD / 2 : 1);
    }
    const bool rot_on = ROPE && mi != 2 && t < R / 2 && rot_i < A.rotary / 2;
    const int64_t rot_pos = rot_on ? A.pos[0] : 0;
    const double rot_f = rot_on ? A.inv_freq[rot_i] : 0.0;
    __builtin_amdgcn_sched_barrier(0);
    FusedRaw<DT> raw[U];
    auto load = [&](int p0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            int b, r;
            if constexpr (SHARED) {
                const int pb = min(p0 + U * g, np - U);
                b = pb / R;
                r = min(pb - b * R + u, rlast);
            } else {
                const int p = min(p0 + U * g + u, np - 1);
                b = p / R;
                r = min(p - b * R, rlast);
            }
            const uint32_t off = tadj + (uint32_t)(fused_row<RD>(A, mi, tile, R, r) - rbase) * rb32 + (uint32_t)b * BYTES;
            if constexpr (DT == DT_Q4_K) {
                raw[u].hdr = *(const u32x4*)(Wt + off);
                raw[u].qv = *(const u32x4*)(Wt + (off + 16 * l + 16));
            } else {
                raw[u].raw = q6k_load_at(Wt, off, l);
            }
        }
    };
    load(0);
    __builtin_amdgcn_sched_barrier(0);

    // 2. Quantize x (NORM: rms_norm(x + resid) * scale) into LDS while the
    // weights arrive (lead team; the others wait at its barrier).
    bool bad = false;
    if constexpr (NORM) {
        if (lead) bad = norm_quantize_lds<NORM_KL<TEAMS>>(A, N, blockIdx.x == 0, yl, npart, Q);
        else bad = norm_quantize_helper<NORM_PER<TEAMS>>(A, N, NORM_KL<TEAMS> + (team - 1) * NORM_PER<TEAMS>, yl, npart, Q);
    } else if (lead) {
        bad = bq < nb ? quantize_block_lds(xv, bq, j, Q) : false;
        for (int b = bq + 16; b < nb; b += 16) {  // rows longer than 4096
            load_x16(A.x, b, j, xv);
            bad |= quantize_block_lds(xv, b, j, Q);
        }
    }
    // (one LDS barrier, not HIP's three of __syncthreads_or after a wait for
    // every load in flight: measured on MI355X, 8B decode batch 1 +1.7 %,
    // the cfg1 layer set 0.5 % slower)
    const bool row_refused = wg_any(bad, wflag, nwaves);

    // (rope: the rotation of this thread's pair, while the weights arrive)
    float rc = 1.f, rs = 0.f;
    if (rot_on) {
        const double ang = (double)rot_pos * rot_f;
        rc = (float)cos(ang);
        rs = (float)sin(ang);
    }

    // 3. Exact block sums of this workgroup's pairs.
    for (int p0 = 0; p0 < np; p0 += 32 * U) {
        if (p0 != 0) load(p0);
        const int pb = p0 + U * g;
        ActLane a0;
        if constexpr (SHARED) a0 = act_lane_lds<DT>(Q, min(pb, np - U) / R, l);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int p = SHARED ? min(pb, np - U) + u : min(pb + u, np - 1);
            const bool store = SHARED ? pb < np : pb + u < np;
            const int b = p / R, r = p - b * R;
            const ActLane a = SHARED ? a0 : act_lane_lds<DT>(Q, b, l);
            u32x4 hdr = {0, 0, 0, 0}, qv = {0, 0, 0, 0};
            Q6KRaw q6{};
            if constexpr (DT == DT_Q4_K) {
                hdr = raw[u].hdr;
                qv = raw[u].qv;
            } else {
                q6 = raw[u].raw;
            }
            const i32x4 v = pair_part<DT>(hdr, qv, q6, a, l);
            if (l == 0 && store) part[r * nb + b] = v;
        }
    }
    if (t < R) refl[t] = wr;
    __syncthreads();

    // 4. The serial float chain of each row, in block order.
    if (t < R) {
        const int row = fused_row<RD>(A, mi, tile, R, t);
        if (row0 + t < F.N && wr == 0 && !row_refused) {
            float tot = 0.f, off = 0.f;
            for (int b = 0; b < nb; b++) {
                const i32x4 v = part[t * nb + b];
                tot = __builtin_fmaf((float)v.x, __int_as_float(v.z), tot);
                if (DT == DT_Q4_K) off = __builtin_fmaf((float)v.y, __int_as_float(v.w), off);
            }
            float res = DT == DT_Q4_K ? tot - off : tot;
            if (F.bias) res += bias;
            if (ROPE) yr[t] = res;
            else F.y[row] = res;
        }
    }
    // 5. The float32 path for refused rows (fused order: one activation row).
    for (int r = g; r < R; r += 32) {
        const int row = fused_row<RD>(A, mi, tile, R, r);
        if (row0 + r < F.N && (refl[r] != 0 || row_refused)) {
            float res = f32dot_g8<DT>(F.W + (int64_t)row * F.rb, NORM ? (const float*)yl : A.x, K, true);
            if (F.bias) res += F.bias[row];
            if (l == 0) {
                if (ROPE) yr[r] = res;
                else F.y[row] = res;
            }
        }
    }
    if constexpr (!ROPE) return;
    // 6. rope.v1 and the cache scatter (rope_kv_kernel's steps, T = 1): q
    // rotated to y, k rotated and v to the caches at cidx[0].
    __syncthreads();
    const int64_t p = pidx;
    if (mi == 2) {
        const int row = row0 + t;
        if (t < R && row < F.N && p >= 0 && p < A.C) {
            const int hk = row / RD, dd = row - hk * RD;
            const int64_t at = vcache_at(hk, p, dd, RD, A.C);
            if (A.f16) ((_Float16*)A.vc)[at] = (_Float16)yr[t];
            else ((float*)A.vc)[at] = yr[t];
        }
        return;
    }
    if (t < R / 2) {
        constexpr int half = RD / 2;
        const int P = tile * (R / 2) + t, hh = P / half, i = P - hh * half;
        const int ra = fused_row<RD>(A, mi, tile, R, 2 * t), rbb = fused_row<RD>(A, mi, tile, R, 2 * t + 1);
        float xa = yr[2 * t], xb = yr[2 * t + 1];
        if (i < A.rotary / 2) {
            const float x1 = xa, x2 = xb;
            xa = x1 * rc - x2 * rs;
            xb = x2 * rc + x1 * rs;
        }
        if (mi == 0) {
            F.y[ra] = xa;
            F.y[rbb] = xb;
        } else if (p >= 0 && p < A.C) {
            const int64_t at = ((int64_t)hh * A.C + p) * RD;
            const int da = ra - hh * RD, db = rbb - hh * RD;
            if (A.f16) {
                ((_Float16*)A.kc)[at + da] = (_Float16)xa;
                ((_Float16*)A.kc)[at + db] = (_Float16)xb;
            } else {
                ((float*)A.kc)[at + da] = xa;
                ((float*)A.kc)[at + db] = xb;
            }
        }
    }
}

// TEAMS tiles per workgroup (the launch gives every workgroup TEAMS whole
// tiles): team k of workgroup w runs tile TEAMS*w + k.
template <int U, bool SHARED, bool NORM, int RD = 0, int TEAMS = 1>
__global__ __launch_bounds__(256 * TEAMS) void gemv_a8k_fused_kernel(FusedArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double npart[4];
    __shared__ int wflag[4 * TEAMS];
    // (a scalar: the lead team's branches around its barrier are uniform
    // jumps, so each wave runs exactly one side and one s_barrier)
    const int team = TEAMS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
    const int gt = (int)blockIdx.x * TEAMS + team;
    int mi = 0;
    if (A.nmat > 1 && gt >= A.mat[1].tile0) mi = 1;
    if (A.nmat > 2 && gt >= A.mat[2].tile0) mi = 2;
    const FusedMat F = mi == 0 ? A.mat[0] : mi == 1 ? A.mat[1] : A.mat[2];
    const int tile = gt - F.tile0;
    uint8_t* tmem = smem + A.lds_row + (size_t)team * A.lds_team;
    if (F.dt == DT_Q4_K)
        fused_body<DT_Q4_K, U, SHARED, NORM, RD, TEAMS>(A, F, mi, tile, smem, tmem, npart, wflag, team);
    else fused_body<DT_Q6_K, U, SHARED, NORM, RD, TEAMS>(A, F, mi, tile, smem, tmem, npart, wflag, team);
}

// LDS of the shared row: q, dx, xs, ys16 (and the normed row, K floats).
static size_t fused_lds_row(int64_t K, int nb, bool norm) {
    const size_t q = ((size_t)K + nb * 4 + (K / 32) * 2 + (K / 16) * 2 + 15) & ~(size_t)15;
    return q + (norm ? (size_t)K * 4 : 0);
}
// LDS of one team: the pair table, the row flags, the rope epilogue's row values.
static size_t fused_lds_team(int nb, int maxR) {
    const size_t base = (size_t)maxR * nb * 16 + (size_t)maxR * 4;
    return (((base + 15) & ~(size_t)15) + (size_t)maxR * 4 + 15) & ~(size_t)15;
}
static size_t fused_lds_bytes(int64_t K, int nb, int maxR, bool norm = false, int teams = 1) {
    return fused_lds_row(K, nb, norm) + (size_t)teams * fused_lds_team(nb, maxR);
}

// Tiles per workgroup: teams share one quantization of the row, so a
// workgroup of three (or two) teams re-reads x (and resid, scale) once for
// three tiles. Taken only where the workgroups still cover every CU.
static int fused_teams(int tiles) {
    if (tiles >= 3 * 256 && tiles % 3 == 0) return 3;
    if (tiles >= 2 * 256 && tiles % 2 == 0) return 2;
    return 1;
}

// Rows per workgroup for a matrix: pairs per workgroup at most 32*U*2 (two
// load batches) and the pair table plus the quantized row within 48 KB.
static int fused_rows(int nb, int64_t K) {
    constexpr int U = 4;
    int R = max(1, 32 * U / nb);
    while (R > 1 && fused_lds_bytes(K, nb, R) > 48 * 1024) R >>= 1;
    return R;
}

bool fused_gemv_ok(const DevWeight* const* ws, int nmat) {
    if (nmat < 1 || nmat > 3) return false;
    const int64_t K = ws[0]->k;
    if (K % 256 || K > 16384) return false;
    for (int i = 0; i < nmat; i++)
        if (ws[i]->k != K || (ws[i]->dt != DT_Q4_K && ws[i]->dt != DT_Q6_K)) return false;
    return fused_lds_bytes(K, (int)(K / 256), fused_rows((int)(K / 256), K)) <= 48 * 1024;
}

static hipError_t launch_fused(const DevWeight* const* ws, int nmat, const float* x, const float* resid,
                               const float* scale, float eps, float* x_out, bool norm, const float* const* bias,
                               float* const* y, hipStream_t stream, const FusedRope* rope = nullptr) {
    if (!fused_gemv_ok(ws, nmat)) return hipErrorInvalidValue;
    FusedArgs A;
    A.nmat = nmat;
    A.x = x;
    A.resid = resid;
    A.scale = scale;
    A.eps = eps;
    A.x_out = x_out;
    A.rope = 0;
    A.pos = A.cidx = nullptr;
    A.inv_freq = nullptr;
    A.D = A.rotary = A.interleaved = A.f16 = 0;
    A.C = 0;
    A.kc = A.vc = nullptr;
    if (rope) {
        A.rope = 1;
        A.pos = rope->pos;
        A.cidx = rope->cidx;
        A.inv_freq = rope->inv_freq;
        A.D = rope->d;
        A.rotary = rope->rotary;
        A.interleaved = rope->interleaved;
        A.f16 = rope->f16;
        A.C = rope->context;
        A.kc = rope->kcache;
        A.vc = rope->vcache;
    }
    A.K = ws[0]->k;
    A.nb = (int)(A.K / 256);
    int tiles = 0, maxR = 1;
    for (int i = 0; i < 3; i++) {
        FusedMat& F = A.mat[i];
        const DevWeight& w = *ws[i < nmat ? i : 0];
        F.W = w.data;
        F.wref = w.wref;
        F.bias = i < nmat ? bias[i] : nullptr;
        F.y = i < nmat ? y[i] : nullptr;
        F.rb = w.row_bytes;
        F.N = (int)w.n;
        F.dt = w.dt;
        F.R = fused_rows(A.nb, A.K);
        F.tile0 = tiles;
        if (i < nmat) {
            tiles += (F.N + F.R - 1) / F.R;
            maxR = max(maxR, F.R);
        }
    }
    const int teams = fused_teams(tiles);
    A.lds_row = (int)fused_lds_row(A.K, A.nb, norm);
    A.lds_team = (int)fused_lds_team(A.nb, maxR);
    const size_t lds = fused_lds_bytes(A.K, A.nb, maxR, norm, teams);
    const dim3 grid(tiles / teams), block(256 * teams);
    // every matrix has the same R (it depends on K only)
    const bool shared = A.mat[0].R % 4 == 0;
#define MIMG_FUSED_LAUNCH(SH, NO, RD_)                                                                              \
    do {                                                                                                           \
        if (teams == 3) hipLaunchKernelGGL((gemv_a8k_fused_kernel<4, SH, NO, RD_, 3>), grid, block, lds, stream, A); \
        else if (teams == 2)                                                                                       \
            hipLaunchKernelGGL((gemv_a8k_fused_kernel<4, SH, NO, RD_, 2>), grid, block, lds, stream, A);           \
        else hipLaunchKernelGGL((gemv_a8k_fused_kernel<4, SH, NO, RD_, 1>), grid, block, lds, stream, A);          \
    } while (0)
    if (rope) {
        if (!norm || !shared || (rope->d != 64 && rope->d != 128)) return hipErrorInvalidValue;
        if (rope->d == 64) MIMG_FUSED_LAUNCH(true, true, 64);
        else MIMG_FUSED_LAUNCH(true, true, 128);
    } else if (norm && shared) MIMG_FUSED_LAUNCH(true, true, 0);
    else if (norm) MIMG_FUSED_LAUNCH(false, true, 0);
    else if (shared) MIMG_FUSED_LAUNCH(true, false, 0);
    else MIMG_FUSED_LAUNCH(false, false, 0);
#undef MIMG_FUSED_LAUNCH
    return hipGetLastError();
}

hipError_t launch_gemv_a8k_fused(const DevWeight* const* ws, int nmat, const float* x,
                                 const float* const* bias, float* const* y, hipStream_t stream) {
    return launch_fused(ws, nmat, x, nullptr, nullptr, 0.f, nullptr, false, bias, y, stream);
}

bool fused_norm_ok(const DevWeight* const* ws, int nmat) {
    const int64_t K = ws[0]->k;
    return fused_gemv_ok(ws, nmat) && K % 1024 == 0 && K <= 256 * 4 * NORM_R &&
           fused_lds_bytes(K, (int)(K / 256), fused_rows((int)(K / 256), K), true) <= 64 * 1024;
}

hipError_t launch_gemv_a8k_fused_norm(const DevWeight* const* ws, int nmat, const float* x, const float* resid,
                                      const float* scale, float eps, float* x_out, const float* const* bias,
                                      float* const* y, hipStream_t stream) {
    if (!fused_norm_ok(ws, nmat) || !x_out) return hipErrorInvalidValue;
    return launch_fused(ws, nmat, x, resid, scale, eps, x_out, true, bias, y, stream);
}

// q, k, v with rope and the cache scatter in the epilogue: each workgroup's
// rows must be whole rotation pairs of one head.
bool fused_norm_rope_ok(const DevWeight* const* ws, int heads, int kv_heads, int d, int rotary) {
    if (!fused_norm_ok(ws, 3) || (d != 64 && d != 128) || rotary <= 0 || rotary % 2 || rotary > d) return false;
    const int64_t K = ws[0]->k;
    const int R = fused_rows((int)(K / 256), K);
    if (R % 4 || (d / 2) % (R / 2)) return false;
    return ws[0]->n == (int64_t)heads * d && ws[1]->n == (int64_t)kv_heads * d && ws[2]->n == (int64_t)kv_heads * d;
}

hipError_t launch_gemv_a8k_fused_norm_rope(const DevWeight* const* ws, const float* x, const float* resid,
                                           const float* scale, float eps, float* x_out, const float* const* bias,
                                           float* q, const FusedRope& rope, hipStream_t stream) {
    if (!fused_norm_rope_ok(ws, rope.heads, rope.kv_heads, rope.d, rope.rotary) || !x_out) return hipErrorInvalidValue;
    float* y[3] = {q, nullptr, nullptr};
    return launch_fused(ws, 3, x, resid, scale, eps, x_out, true, bias, y, stream, &rope);
}

}  // namespace mimg
