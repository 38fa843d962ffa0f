// The ops around the linear layers in a llama/qwen2 decoder step, on the
// GPU so that a step's activations stay in device memory: the other fast
// paths of the graph BuildLlama writes (reference importer/llama.go:317-547,
// interp/fast.go:40-59). Their float results follow the reference's
// formulas and, for attention and swiglu, the operation order of the AVX2
// kernels the reference runs on amd64; the f64 steps (rms_norm's sum of
// squares, rope's cos/sin, the exp of tails) round to the same f32 except
// with probability ~1e-7 per value (another f64 summation order or libm).
//
//   embedding.v1  rows of the table decoded exactly (interp/fast.go:818-842)
//   rms_norm.v1   f64 sum of squares; inv = f32(1/sqrt(f64(f32(ss/n)) +
//                 f64(f32(eps)))); y = (x*inv)*scale (interp/fast.go:434-485)
//   rope.v1       angles pos*invFreq_i in f64, c = f32(cos), s = f32(sin),
//                 x1*c - x2*s, x2*c + x1*s in f32 (interp/fast.go:507-557)
//   attention.v1/2  keys j <= position visible; attendRow in the order of the
//                 reference's AVX2 kernels (interp/fast.go:728-751,
//                 attn_amd64.s): bit for bit; with the cache in f16, keys
//                 and values are rounded to f16 as they are stored
//   swiglu.v1     SiluMulF32 over the reference's pieces (fast.go:487-498,
//                 attn.go:63-76, attn_amd64.s:459-535): bit for bit
//   argmax        first index of the largest logit (cmd/mim-run/main.go:184-192)
#include <type_traits>

#include "decoder_math.hpp"
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// Rows of the embedding table for the given tokens: out[t][e].
template <uint32_t DT>
__global__ void embed_rows_kernel(const uint8_t* __restrict__ table, int64_t row_bytes, const int32_t* __restrict__ ids,
                                  int V, int64_t E, float* __restrict__ out) {
    const int t = blockIdx.y;
    const int id = ids[t];
    // Out-of-range ids give a zero row, as the reference's gather leaves
    // them (interp/fast.go:834-838); no table byte is read for them.
    const bool valid = id >= 0 && id < V;
    const uint8_t* row = table + (int64_t)(valid ? id : 0) * row_bytes;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < E; e += (int64_t)gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (valid) {
            if constexpr (DT == DT_F32) v = ((const float*)row)[e];
            else v = decode_weight<DT>(row, e);
        }
        out[(int64_t)t * E + e] = v;
    }
}

// One 256-thread workgroup per row: x += resid (if given, written back to
// x), then y = rms_norm(x) * scale. Rows of up to RMS_REG*256*4 elements
// with n % 4 == 0 are held in registers (one pass over memory); longer or
// ragged rows take a second pass.
constexpr int RMS_REG = 8;
__global__ __launch_bounds__(256) void rms_norm_kernel(float* __restrict__ x, const float* __restrict__ resid,
                                                       const float* __restrict__ scale, float eps, int64_t n,
                                                       float* __restrict__ y) {
    __shared__ double part[4];
    float* xr = x + (int64_t)blockIdx.x * n;
    const float* rr = resid ? resid + (int64_t)blockIdx.x * n : nullptr;
    float* yr = y + (int64_t)blockIdx.x * n;
    const int tid = threadIdx.x;
    const bool inreg = n % 4 == 0 && n <= (int64_t)RMS_REG * 256 * 4;
    float4 v[RMS_REG];
    double ss = 0.0;
    if (inreg) {
        const int64_t n4 = n / 4;
#pragma unroll
        for (int k = 0; k < RMS_REG; k++) {
            const int64_t i = tid + 256 * k;
            if (i < n4) {
                v[k] = ((const float4*)xr)[i];
                if (rr) {
                    const float4 r4 = ((const float4*)rr)[i];
                    v[k].x = v[k].x + r4.x;
                    v[k].y = v[k].y + r4.y;
                    v[k].z = v[k].z + r4.z;
                    v[k].w = v[k].w + r4.w;
                    ((float4*)xr)[i] = v[k];
                }
                ss += (double)v[k].x * (double)v[k].x + (double)v[k].y * (double)v[k].y +
                      (double)v[k].z * (double)v[k].z + (double)v[k].w * (double)v[k].w;
            }
        }
    } else {
        for (int64_t i = tid; i < n; i += 256) {
            float e = xr[i];
            if (rr) {
                e = e + rr[i];
                xr[i] = e;
            }
            ss += (double)e * (double)e;
        }
    }
    ss = wave_sum_f64(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = (float)(1.0 / sqrt((double)(float)(tot / (double)n) + (double)eps));
    if (inreg) {
        const int64_t n4 = n / 4;
#pragma unroll
        for (int k = 0; k < RMS_REG; k++) {
            const int64_t i = tid + 256 * k;
            if (i < n4) {
                float4 o = {v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv};
                if (scale) {
                    const float4 s4 = ((const float4*)scale)[i];
                    o.x = o.x * s4.x;
                    o.y = o.y * s4.y;
                    o.z = o.z * s4.z;
                    o.w = o.w * s4.w;
                }
                ((float4*)yr)[i] = o;
            }
        }
    } else {
        for (int64_t i = tid; i < n; i += 256) {
            const float e = xr[i] * inv;
            yr[i] = scale ? e * scale[i] : e;
        }
    }
}

// x [T][heads][D] rotated in place; inv_freq [rotary/2] in f64.
__global__ void rope_kernel(float* __restrict__ x, const int64_t* __restrict__ pos, const double* __restrict__ inv_freq,
                            int T, int heads, int D, int rotary, int interleaved) {
    const int h2 = rotary / 2;
    const int64_t total = (int64_t)T * heads * h2;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % h2);
        const int64_t th = idx / h2;
        const int t = (int)(th / heads);
        const double ang = (double)pos[t] * inv_freq[i];
        const float c = (float)cos(ang), s = (float)sin(ang);
        float* row = x + th * D;
        const int i1 = interleaved ? 2 * i : i, i2 = interleaved ? 2 * i + 1 : i + h2;
        const float x1 = row[i1], x2 = row[i2];
        const float a = x1 * c, b = x2 * s, cc = x2 * c, d = x1 * s;
        row[i1] = a - b;
        row[i2] = cc + d;
    }
}


// k, v [T][Hkv][D] into the caches at the cache indices pos[t] (rounded to
// f16 when the cache is f16).
__global__ void kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v, const int64_t* __restrict__ pos,
                                int T, int Hkv, int D, int64_t C, void* kc, void* vc, int f16) {
    const int64_t total = (int64_t)T * Hkv * D;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(idx % D);
        const int64_t th = idx / D;
        const int hk = (int)(th % Hkv), t = (int)(th / Hkv);
        const int64_t p = pos[t];
        if (p < 0 || p >= C) continue;  // outside the cache: not stored
        const int64_t at = ((int64_t)hk * C + p) * D + d, av = vcache_at(hk, p, d, D, C);
        if (f16) {
            ((_Float16*)kc)[at] = (_Float16)k[idx];
            ((_Float16*)vc)[av] = (_Float16)v[idx];
        } else {
            ((float*)kc)[at] = k[idx];
            ((float*)vc)[av] = v[idx];
        }
    }
}


// rope.v1 on q and k and the cache scatter of k and v in one launch (the
// graph's rope of q and k and its cache update, importer/llama.go:364-503):
// a workgroup per (row t, head), heads 0..H-1 of q, then Hkv of k, then Hkv
// of v; thread i takes one pair of dims: (2i, 2i+1) when interleaved, else
// (i, i + rotary/2) for i < rotary/2 and two adjacent dims past the rotary
// ones. q is rotated in place; k (rotated) and v go to the caches at cidx[t]
// (rounded to f16 with an f16 cache; rows outside the cache are not stored).
template <bool F16>
__global__ void rope_kv_kernel(float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                               const int64_t* __restrict__ pos, const int64_t* __restrict__ cidx,
                               const double* __restrict__ inv_freq, int H, int Hkv, int D, int rotary, int interleaved,
                               int64_t C, void* kc, void* vc) {
    const int t = blockIdx.y, hh = blockIdx.x, i = threadIdx.x;
    if (i >= D / 2) return;
    const int h2 = rotary / 2;
    int a, b;
    if (interleaved) {
        a = 2 * i;
        b = 2 * i + 1;
    } else if (i < h2) {
        a = i;
        b = i + h2;
    } else {
        a = rotary + 2 * (i - h2);
        b = a + 1;
    }
    const bool rot = i < h2;
    float* row;
    const float* src;
    if (hh < H) {
        row = q + ((int64_t)t * H + hh) * D;
        src = row;
    } else if (hh < H + Hkv) {
        row = nullptr;
        src = k + ((int64_t)t * Hkv + (hh - H)) * D;
    } else {
        row = nullptr;
        src = v + ((int64_t)t * Hkv + (hh - H - Hkv)) * D;
    }
    float xa = src[a], xb = src[b];
    if (rot && hh < H + Hkv) {
        const double ang = (double)pos[t] * inv_freq[i];
        const float c = (float)cos(ang), sn = (float)sin(ang);
        const float x1 = xa, x2 = xb;
        xa = x1 * c - x2 * sn;
        xb = x2 * c + x1 * sn;
    }
    if (row) {
        row[a] = xa;
        row[b] = xb;
        return;
    }
    const int64_t p = cidx[t];
    if (p < 0 || p >= C) return;
    const bool isk = hh < H + Hkv;
    const int hk = isk ? hh - H : hh - H - Hkv;
    const int64_t at = ((int64_t)hk * C + p) * D;
    const int64_t ia = isk ? at + a : vcache_at(hk, p, a, D, C), ib = isk ? at + b : vcache_at(hk, p, b, D, C);
    void* cache = isk ? kc : vc;
    if constexpr (F16) {
        ((_Float16*)cache)[ia] = (_Float16)xa;
        ((_Float16*)cache)[ib] = (_Float16)xb;
    } else {
        ((float*)cache)[ia] = xa;
        ((float*)cache)[ib] = xb;
    }
}

// attention.v1/.v2 in the reference's attendRow order (interp/fast.go:728-751
// with attn_amd64.s), bit for bit, as two kernels:
//   att_scores  a workgroup per (64-key tile, head h, query t): eight lanes
//               per key, lane c sums q[8m+c]*k[8m+c] by fma over m; keys go
//               in fours from the first visible one, reduced
//               ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)), the last n%4 keys as
//               ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)); times scale; into the
//               workspace row of (t, h)
//   att_wsum    a workgroup per (slice of DS dims, head h, query t): max,
//               Cephes exp of s - max for the first n&~7 keys (eight
//               stride-8 lane sums in key order, then HSUM), the f64 exp
//               for the tail added in order; then for each dim d of the
//               slice acc = fma(e_j, v_j[d], acc) over the keys in order
//               (the values staged through LDS, as many keys at a time as
//               fit beside the scores in 64 KB), and
//               o[d] = acc / sum
// The visible keys of query t are cache entries kstart[t]..kend[t] (kstart
// 0 when null) of kv head h / (H / Hkv), clipped to the cache row and to
// maxk (the workspace row). A non-finite largest score gives NaN (the
// reference's scalar loop ends in NaN then); no visible key gives zeros.
constexpr int ATT_MAXC = 8192;

struct AttRange {
    int64_t k0, n;
};
__device__ __forceinline__ AttRange att_range(const int64_t* kend, const int64_t* kstart, int t, int64_t C,
                                              int64_t maxk) {
    AttRange r;
    r.k0 = kstart ? (kstart[t] < 0 ? 0 : (kstart[t] >= C ? C - 1 : kstart[t])) : 0;
    int64_t n = kend[t] + 1 - r.k0;
    if (n > C - r.k0) n = C - r.k0;
    if (n > maxk) n = maxk;
    r.n = n < 0 ? 0 : n;
    return r;
}

template <bool F16>
__device__ __forceinline__ float kv_load(const void* c, int64_t i) {
    if constexpr (F16) return (float)((const _Float16*)c)[i];
    else return ((const float*)c)[i];
}

// The score of one key from the eight lanes' chains l (lane c of the group
// holds l_c): ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)) for keys in the groups of
// four, ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) for the last n%4; lane 0 of the
// group returns it.
// The partner values move by DPP within each group of eight lanes: lane
// c ^ 1 and c ^ 2 by quad permutes, c ^ 4 by row shifts of four into the
// upper and the lower half-group (bank masks). Float addition commutes, so
// every lane of the group ends with the same sum.
__device__ __forceinline__ float xchg1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_QUAD_1032, 0xF, 0xF, false));
}
__device__ __forceinline__ float xchg2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_QUAD_2301, 0xF, 0xF, false));
}
__device__ __forceinline__ float xchg4(float v) {
    constexpr int ROW_SHL4 = 0x104, ROW_SHR4 = 0x114;
    const int x = __float_as_int(v);
    int t = __builtin_amdgcn_update_dpp(x, x, ROW_SHR4, 0xF, 0xA, false);  // lanes 4-7, 12-15 of a row: lane - 4
    t = __builtin_amdgcn_update_dpp(t, x, ROW_SHL4, 0xF, 0x5, false);      // lanes 0-3, 8-11: lane + 4
    return __int_as_float(t);
}
__device__ __forceinline__ float att_reduce8(float l, bool four, int gbase, int c) {
    (void)gbase;
    (void)c;
    const float a = l + xchg1(l), b = a + xchg2(a);
    const float pf = b + xchg4(b);  // ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7))
    if (__all(four)) return pf;
    const float e = l + xchg4(l), f = e + xchg1(e);
    const float pn = f + xchg2(f);  // ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7))
    return four ? pf : pn;
}

// DM = D/8 for D = 64 or 128 (unrolled; every load of a lane in flight at
// once), 0 for other multiples of 8. QT queries per workgroup (rows
// QT*z .. QT*z + QT-1 of T): when they share the first visible cache entry
// (rows of one sequence), each key is loaded once for all of them.
template <bool F16, int DM, int QT>
__global__ __launch_bounds__(256) void att_scores_kernel(const float* __restrict__ q, const void* kc,
                                                         const int64_t* __restrict__ kend,
                                                         const int64_t* __restrict__ kstart, int T, int H, int Hkv,
                                                         int D, int64_t C, int64_t maxk, float* __restrict__ ws) {
    const int tile = blockIdx.x, h = blockIdx.y;
    AttRange r[QT];
    int64_t nmax = 0;
#pragma unroll
    for (int i = 0; i < QT; i++) {
        const int t = QT * blockIdx.z + i;
        r[i] = t < T ? att_range(kend, kstart, t, C, maxk) : AttRange{0, 0};
        nmax = r[i].n > nmax ? r[i].n : nmax;
    }
    if ((int64_t)tile * 64 >= nmax) return;
    int i0 = 0;  // the first query with keys (nmax > 0)
    while (r[i0].n == 0) i0++;
    bool same = true;
#pragma unroll
    for (int i = 0; i < QT; i++) same = same && (r[i].n == 0 || r[i].k0 == r[i0].k0);
    const int hk = h / (H / Hkv);
    const int lane = threadIdx.x & 63, c = lane & 7, gbase = lane & ~7, grp = threadIdx.x >> 3;
    const float scale = (float)(1.0 / sqrt((double)D));
    const int64_t j0 = (int64_t)tile * 64 + grp, j1 = j0 + 32;
    constexpr int DMR = DM > 0 ? DM : 1;
    // one query: dot products of q with keys at a0, a1 (cache entries)
    auto query_scores = [&](int i, const float* kv0, const float* kv1, int64_t a0, int64_t a1) {
        const int t = QT * blockIdx.z + i;
        const float* qr = q + ((int64_t)t * H + h) * D;
        float l0 = 0.f, l1 = 0.f;
        if constexpr (DM > 0) {
#pragma unroll
            for (int m = 0; m < DM; m++) {
                const float qm = qr[8 * m + c];
                l0 = __builtin_fmaf(qm, kv0[m], l0);
                l1 = __builtin_fmaf(qm, kv1[m], l1);
            }
        } else {
            for (int m = 0; m < D / 8; m++) {
                const float qm = qr[8 * m + c];
                l0 = __builtin_fmaf(qm, kv_load<F16>(kc, a0 * D + 8 * m + c), l0);
                l1 = __builtin_fmaf(qm, kv_load<F16>(kc, a1 * D + 8 * m + c), l1);
            }
        }
        const int64_t n = r[i].n, n4 = n - n % 4;
        const float p0 = att_reduce8(l0, j0 < n4, gbase, c);
        const float p1 = att_reduce8(l1, j1 < n4, gbase, c);
        float* out = ws + ((int64_t)t * H + h) * maxk;
        if (c == 0) {
            if (j0 < n) out[j0] = p0 * scale;
            if (j1 < n) out[j1] = p1 * scale;
        }
    };
    auto load_keys = [&](int64_t base, int64_t n, float* kv0, float* kv1, int64_t& a0, int64_t& a1) {
        // past the end the last key is recomputed, unstored
        a0 = base + (j0 < n ? j0 : n - 1);
        a1 = base + (j1 < n ? j1 : n - 1);
        if constexpr (DM > 0) {
#pragma unroll
            for (int m = 0; m < DM; m++) {
                kv0[m] = kv_load<F16>(kc, a0 * D + 8 * m + c);
                kv1[m] = kv_load<F16>(kc, a1 * D + 8 * m + c);
            }
        }
    };
    float kv0[DMR], kv1[DMR];
    int64_t a0, a1;
    if (same) {
        load_keys((int64_t)hk * C + r[i0].k0, nmax, kv0, kv1, a0, a1);
#pragma unroll
        for (int i = 0; i < QT; i++)
            if ((int64_t)tile * 64 < r[i].n) query_scores(i, kv0, kv1, a0, a1);
    } else {
        for (int i = 0; i < QT; i++) {
            if ((int64_t)tile * 64 >= r[i].n) continue;
            load_keys((int64_t)hk * C + r[i].k0, r[i].n, kv0, kv1, a0, a1);
            query_scores(i, kv0, kv1, a0, a1);
        }
    }
}

// Decode scores with grouped-query heads: a workgroup per (64 keys, kv
// head, query) computes the scores of the G query heads that share the kv
// head, each key loaded once for all G (att_scores_kernel loads it once per
// query head). Every score's float steps are att_scores_kernel's (eight
// lanes per key, lane c's fma chain over m, att_reduce8's pairing, times the
// scale), so the results are bit for bit the same. The G heads' q rows are
// loaded first (L2-resident), then the keys.
template <bool F16, int DM, int G>
__global__ __launch_bounds__(256) void att_scores_gqa_kernel(const float* __restrict__ q, const void* kc,
                                                             const int64_t* __restrict__ kend,
                                                             const int64_t* __restrict__ kstart, int T, int H, int Hkv,
                                                             int D, int64_t C, int64_t maxk, float* __restrict__ ws) {
    const int tile = blockIdx.x, hk = blockIdx.y, t = blockIdx.z;
    const AttRange r = att_range(kend, kstart, t, C, maxk);
    const int64_t n = r.n;
    if ((int64_t)tile * 64 >= n) return;
    const int lane = threadIdx.x & 63, c = lane & 7, gbase = lane & ~7, grp = threadIdx.x >> 3;
    const float scale = (float)(1.0 / sqrt((double)D));
    float qv[G][DM];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const float* qr = q + ((int64_t)t * H + hk * G + gi) * D;
#pragma unroll
        for (int m = 0; m < DM; m++) qv[gi][m] = qr[8 * m + c];
    }
    const int64_t j0 = (int64_t)tile * 64 + grp, j1 = j0 + 32;
    const int64_t base = (int64_t)hk * C + r.k0;
    const int64_t a0 = base + (j0 < n ? j0 : n - 1), a1 = base + (j1 < n ? j1 : n - 1);  // past the end: the last key
    float kv0[DM], kv1[DM];
#pragma unroll
    for (int m = 0; m < DM; m++) {
        kv0[m] = kv_load<F16>(kc, a0 * D + 8 * m + c);
        kv1[m] = kv_load<F16>(kc, a1 * D + 8 * m + c);
    }
    const int64_t n4 = n - n % 4;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int m = 0; m < DM; m++) {
            l0 = __builtin_fmaf(qv[gi][m], kv0[m], l0);
            l1 = __builtin_fmaf(qv[gi][m], kv1[m], l1);
        }
        const float p0 = att_reduce8(l0, j0 < n4, gbase, c);
        const float p1 = att_reduce8(l1, j1 < n4, gbase, c);
        float* out = ws + ((int64_t)t * H + hk * G + gi) * maxk;
        if (c == 0) {
            if (j0 < n) out[j0] = p0 * scale;
            if (j1 < n) out[j1] = p1 * scale;
        }
    }
}

// One query's attention in one launch (decode): a workgroup per (DG dims,
// head, query) computes all of the query's scores itself (the workgroups of
// one head repeat them, each score in the same order), then the softmax and
// the ordered weighted sum of its dims. The steps and their float order are
// those of att_scores_kernel and att_wsum_kernel:
//   score j: lane c of a group of eight runs l_c = fma(q[8m+c], k_j[8m+c],
//     l_c) over m, the group adds the eight as att_reduce8 does (here with
//     DPP moves; only lane 0's sum is used, and its partners are the same),
//     times 1/sqrt(D);
//   max, NaN check, Cephes exp for the first n&~7 keys and the f64 exp for
//   the rest, eight stride-8 lane sums + HSUM + the tail in order;
//   per dim acc = fma(e_j, v_j[d], acc) in key order, then acc / sum.
// Keys are read with one load per lane and element, two keys per group in
// flight while the previous two are summed; the values of the workgroup's
// dims are staged dim-major in LDS from the 8-key block holding the first
// visible key (16 bytes a dim and block); the lane sums (wave 1) run beside
// the chain (wave 0).
// Lane i of a row of 16 reads lane (i - n) mod 16 under row_ror:n, so
// row_ror:12 gives lane i lane i+4 (lanes 0..3 of each group of eight read
// lanes 4..7 of the same group).
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_ROR4 = 0x12C;

__device__ __forceinline__ float dpp_f(float v, int ctrl) {
    const int x = __float_as_int(v);
    switch (ctrl) {
    case DPP_XOR1: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_XOR1, 0xF, 0xF, true));
    case DPP_XOR2: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_XOR2, 0xF, 0xF, true));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROR4, 0xF, 0xF, true));
    }
}

// att_reduce8's sum at lane 0 of each group of eight: with four,
// ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)); otherwise ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)).
// (The row rotation gives lanes 0..3 their partners c+4, all lane 0 needs.)
__device__ __forceinline__ float reduce8_lane0(float l, bool four) {
    float a = l + (four ? dpp_f(l, DPP_XOR1) : dpp_f(l, DPP_ROR4));
    float b = a + (four ? dpp_f(a, DPP_XOR2) : dpp_f(a, DPP_XOR1));
    return b + (four ? dpp_f(b, DPP_ROR4) : dpp_f(b, DPP_XOR2));
}

// Elements per dim row of the staged values: maxk keys from a block start
// (up to 7 more), rounded to blocks of 8, plus 16 bytes so that the lanes'
// rows start in different banks.
template <bool F16>
__host__ __device__ constexpr int64_t att_dec_vstride(int64_t maxk) {
    return ((maxk + 7 + 7) & ~(int64_t)7) + (F16 ? 8 : 4);
}

template <bool F16, int D, int DG>
__global__ __launch_bounds__(256) void att_decode_kernel(const float* __restrict__ q, const void* kc, const void* vc,
                                                         const int64_t* __restrict__ kend,
                                                         const int64_t* __restrict__ kstart, int H, int Hkv, int64_t C,
                                                         int64_t maxk, float* __restrict__ out) {
    extern __shared__ float att_lds[];
    __shared__ float red[4];
    __shared__ float lane_sum[8];
    __shared__ int nan_any;
    using VT = typename std::conditional<F16, _Float16, float>::type;
    constexpr int DM = D / 8;
    constexpr int PER_KEY = DG * (int)sizeof(VT) / 16;  // 16-byte pieces of a key's DG values
    constexpr int VPAD = F16 ? 8 : 4;
    const int d0 = blockIdx.x * DG, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x, w = tid >> 6;
    const int lane = tid & 63, c = lane & 7, grp = tid >> 3;
    const AttRange r = att_range(kend, kstart, t, C, maxk);
    const int64_t n = r.n;
    float* orow = out + ((int64_t)t * H + h) * D + d0;
    if (n <= 0) {
        if (tid < DG) orow[tid] = 0.f;
        return;
    }
    const int hk = h / (H / Hkv);
    const int64_t base = (int64_t)hk * C + r.k0;  // first visible cache row
    const int64_t mk = (maxk + 3) & ~(int64_t)3, vstride = att_dec_vstride<F16>(maxk);
    float* sc = att_lds;            // [mk]: scores, then exponentials
    VT* vb = (VT*)(att_lds + mk);   // [DG][vstride]: values, dim-major from key k0 & ~7
    if (tid == 0) nan_any = 0;

    // 1. Scores: group grp takes keys grp, grp+32, ..., two at a time, the
    // next two's loads issued before the current two are summed.
    const float scale = (float)(1.0 / sqrt((double)D));
    const float* qr = q + ((int64_t)t * H + h) * D;
    float qv[DM];
#pragma unroll
    for (int m = 0; m < DM; m++) qv[m] = qr[8 * m + c];
    const int64_t n4 = n - n % 4;
    float mx = -INFINITY;
    int isnan_local = 0;
    auto kload = [&](int64_t j, float (&kv)[DM]) {
        const int64_t a = base + (j < n ? j : n - 1);  // past the end: the last key, unstored
#pragma unroll
        for (int m = 0; m < DM; m++) kv[m] = kv_load<F16>(kc, a * D + 8 * m + c);
    };
    auto score = [&](int64_t j, const float (&kv)[DM]) {
        float l = 0.f;
#pragma unroll
        for (int m = 0; m < DM; m++) l = __builtin_fmaf(qv[m], kv[m], l);
        const float p = reduce8_lane0(l, j < n4) * scale;
        if (c == 0 && j < n) {
            sc[j] = p;
            isnan_local |= p != p;
            mx = fmaxf(mx, p);
        }
    };
    {
        float ka[DM], kb[DM], kc2[DM], kd[DM];
        int64_t j = grp;
        kload(j, ka);
        kload(j + 32, kb);
        for (; j < n; j += 64) {
            kload(j + 64, kc2);
            kload(j + 96, kd);
            score(j, ka);
            score(j + 32, kb);
#pragma unroll
            for (int m = 0; m < DM; m++) {
                ka[m] = kc2[m];
                kb[m] = kd[m];
            }
        }
    }

    // 2. The values of this workgroup's dims, dim-major into LDS: the 16-byte
    // pieces of (dim, 8-key block) from the block holding key k0, so that
    // key k0 + j of dim d0 + l is vb[l * vstride + off + j].
    const int64_t k0a = r.k0 & ~(int64_t)7, off = r.k0 - k0a, nblk = (off + n + 7) >> 3;
    constexpr int PPB = F16 ? 1 : 2;  // 16-byte pieces per (dim, block)
    const VT* vsrc = (const VT*)vc + vcache_at(hk, k0a, d0, D, C);
    for (int64_t i = tid; i < nblk * DG * PPB; i += 256) {
        const int64_t jb = i / (DG * PPB);
        const int rem = (int)(i - jb * (DG * PPB)), dl = rem / PPB, pc = rem - dl * PPB;
        const uint4 raw = *(const uint4*)(vsrc + (jb * D + dl) * 8 + pc * 4);
        *(uint4*)(vb + dl * vstride + 8 * jb + pc * 4) = raw;
    }
    (void)PER_KEY;
    (void)base;

    // 3. Max and NaN over the scores, then the exponentials.
    mx = wave_max_f32(mx);
    __syncthreads();  // scores in LDS; nan_any cleared
    if (lane == 0) red[w] = mx;
    if (isnan_local) nan_any = 1;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (nan_any || __builtin_isinf(mx)) {
        if (tid < DG) orow[tid] = __builtin_nanf("");
        return;
    }
    const int64_t nv = n >= 8 ? (n & ~(int64_t)7) : 0;
    for (int64_t j = tid; j < n; j += 256) {
        const float x = sc[j] - mx;
        sc[j] = j < nv ? cephes_exp(x) : (float)exp((double)x);
    }
    __syncthreads();

    // 4. Wave 1: the eight stride-8 lane sums; wave 0: the chain of its dims.
    float acc = 0.f;
    if (w == 1 && lane < 8) {
        float sl = 0.f;
        int64_t j = lane;
        for (; j + 120 < nv; j += 128) {
            float e[16];
#pragma unroll
            for (int u = 0; u < 16; u++) e[u] = sc[j + 8 * u];
#pragma unroll
            for (int u = 0; u < 16; u++) sl = sl + e[u];
        }
        for (; j < nv; j += 8) sl = sl + sc[j];
        lane_sum[lane] = sl;
    } else if (w == 0 && lane < DG) {
        const VT* vd = vb + lane * vstride + off;
        using VR = typename std::conditional<F16, uint2, float4>::type;
        auto fetch = [&](int64_t j, float4 (&ev)[4], VR (&vr)[4]) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                ev[u] = *(const float4*)(sc + j + 4 * u);
                vr[u] = *(const VR*)(vd + j + 4 * u);
            }
        };
        auto chain16 = [&](const float4 (&ev)[4], const VR (&vr)[4]) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float4 vv;
                if constexpr (F16) {
                    vv = make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(vr[u].x & 0xFFFF)),
                                     (float)__builtin_bit_cast(_Float16, (uint16_t)(vr[u].x >> 16)),
                                     (float)__builtin_bit_cast(_Float16, (uint16_t)(vr[u].y & 0xFFFF)),
                                     (float)__builtin_bit_cast(_Float16, (uint16_t)(vr[u].y >> 16)));
                } else {
                    vv = vr[u];
                }
                acc = __builtin_fmaf(ev[u].x, vv.x, acc);
                acc = __builtin_fmaf(ev[u].y, vv.y, acc);
                acc = __builtin_fmaf(ev[u].z, vv.z, acc);
                acc = __builtin_fmaf(ev[u].w, vv.w, acc);
            }
        };
        int64_t j = 0;
        if (n >= 16 && (off & 3) == 0) {  // (values of four keys in one aligned read)
            float4 eA[4], eB[4];
            VR vA[4], vB[4];
            fetch(0, eA, vA);
            for (; j + 32 <= n; j += 32) {
                fetch(j + 16, eB, vB);
                chain16(eA, vA);
                if (j + 48 <= n) fetch(j + 32, eA, vA);
                chain16(eB, vB);
            }
            if (j + 16 <= n) {
                chain16(eA, vA);
                j += 16;
            }
        }
        for (; j < n; j++) acc = __builtin_fmaf(sc[j], (float)vd[j], acc);
    }
    __syncthreads();
    if (w == 0 && lane < DG) {
        float sum = ((lane_sum[0] + lane_sum[4]) + (lane_sum[1] + lane_sum[5])) +
                    ((lane_sum[2] + lane_sum[6]) + (lane_sum[3] + lane_sum[7]));
        for (int64_t j = nv; j < n; j++) sum = sum + sc[j];
        orow[lane] = acc / sum;
    }
}

constexpr int64_t ATT_DEC_MAXK = 256;

template <bool F16, int D>
static size_t att_decode_lds(int64_t maxk) {
    constexpr int DG = 32, ESZ = F16 ? 2 : 4;
    const int64_t mk = (maxk + 3) & ~(int64_t)3;
    return (size_t)(mk * 4 + (int64_t)DG * att_dec_vstride<F16>(maxk) * ESZ);
}

// Eight keys of the ordered weighted sum: acc = fma(e[k], v_k, acc) for k =
// 0..7 in order, v_k the k-th value of the dim's 16 (f16) or 32 (f32, v0
// then v1) bytes; att_vget reads one of them.
template <bool F16>
__device__ __forceinline__ void att_chain8(float& acc, const float* e, uint4 v0, uint4 v1) {
    const float4 ea = *(const float4*)e, eb = *(const float4*)(e + 4);
    if constexpr (F16) {
        // (compiled to fmas with an f16 operand, v_fma_mix_f32: the
        // conversion is exact; the chain runs at the fma's dependent-issue
        // latency, about 10 cycles a key on MI355X, as plain f32 fmas do)
        const uint32_t w[4] = {v0.x, v0.y, v0.z, v0.w};
        const float ev[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc = __builtin_fmaf(ev[2 * k], (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xFFFF)), acc);
            acc = __builtin_fmaf(ev[2 * k + 1], (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16)), acc);
        }
        (void)v1;
    } else {
        acc = __builtin_fmaf(ea.x, __uint_as_float(v0.x), acc);
        acc = __builtin_fmaf(ea.y, __uint_as_float(v0.y), acc);
        acc = __builtin_fmaf(ea.z, __uint_as_float(v0.z), acc);
        acc = __builtin_fmaf(ea.w, __uint_as_float(v0.w), acc);
        acc = __builtin_fmaf(eb.x, __uint_as_float(v1.x), acc);
        acc = __builtin_fmaf(eb.y, __uint_as_float(v1.y), acc);
        acc = __builtin_fmaf(eb.z, __uint_as_float(v1.z), acc);
        acc = __builtin_fmaf(eb.w, __uint_as_float(v1.w), acc);
    }
}
template <bool F16>
__device__ __forceinline__ float att_vget(uint4 v0, uint4 v1, int k) {
    if constexpr (F16) {
        const uint32_t w[4] = {v0.x, v0.y, v0.z, v0.w};
        uint32_t x = w[0];
#pragma unroll
        for (int i = 1; i < 4; i++)
            if (k >> 1 == i) x = w[i];
        return (float)__builtin_bit_cast(_Float16, (uint16_t)((k & 1) ? x >> 16 : x & 0xFFFF));
    } else {
        const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        uint32_t x = w[0];
#pragma unroll
        for (int i = 1; i < 8; i++)
            if (k == i) x = w[i];
        return __uint_as_float(x);
    }
}

// Many queries (prefill): a workgroup per (64 dims, head, four queries),
// wave w for query 4z + w, lane for one dim. The waves share each staged
// chunk of values when their queries share the first visible cache entry;
// otherwise the chunks are staged per query. Per query the steps are those
// of att_wsum_kernel (max, Cephes exp with eight stride-8 lane sums and the
// f64 tail, then acc = fma(e_j, v_j[d], acc) in key order).
// keys per staged chunk of values (a multiple of 8), and elements per dim
// row of the staged chunk: the chunk from the block holding its first key
// (up to 7 more), plus 16 bytes so that the lanes' rows start in different
// banks; 18 KB of LDS
template <bool F16>
constexpr int attq_vc() {
    return F16 ? 128 : 64;
}
template <bool F16>
constexpr int attq_vs() {
    return F16 ? attq_vc<F16>() + 8 : attq_vc<F16>() + 12;  // 68 and 76 dwords: 16 lanes' 16-byte reads hit 64 banks
}

template <bool F16>
__global__ __launch_bounds__(256) void att_wsum_q4_kernel(const void* vc, const int64_t* __restrict__ kend,
                                                          const int64_t* __restrict__ kstart, int T, int H, int Hkv,
                                                          int D, int64_t C, int64_t maxk,
                                                          const float* __restrict__ ws, float* __restrict__ out) {
    extern __shared__ float att_lds[];
    __shared__ int64_t k0s[4], ns[4];
    using VT = typename std::conditional<F16, _Float16, float>::type;
    const int64_t mkp = (maxk + 3) & ~(int64_t)3;
    const int d0 = blockIdx.x * 64, h = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int t = 4 * blockIdx.z + w;
    float* sw = att_lds + w * mkp;
    VT* vb = (VT*)(att_lds + 4 * mkp);
    const AttRange r = t < T ? att_range(kend, kstart, t, C, maxk) : AttRange{0, 0};
    const int64_t n = r.n;
    if (lane == 0) {
        k0s[w] = r.k0;
        ns[w] = n;
    }
    // this wave's scores (eight loads a lane in flight), max and NaN check
    const float* srow = ws + ((int64_t)(t < T ? t : 0) * H + h) * maxk;
    float mx = -INFINITY;
    int bad = 0;
    for (int64_t j0 = lane; j0 < n; j0 += 512) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t j = j0 + 64 * u;
            v[u] = srow[j < n ? j : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t j = j0 + 64 * u;
            if (j < n) {
                sw[j] = v[u];
                bad |= v[u] != v[u];
                mx = fmaxf(mx, v[u]);
            }
        }
    }
    mx = wave_max_f32(mx);
    bad = __any(bad) || __builtin_isinf(mx);
    const int64_t nv = n >= 8 ? (n & ~(int64_t)7) : 0;
    if (!bad)
        for (int64_t j = lane; j < n; j += 64) {
            const float x = sw[j] - mx;
            sw[j] = j < nv ? cephes_exp(x) : (float)exp((double)x);
        }
    __syncthreads();
    float s = 0.f;
    if (lane < 8)
        for (int64_t j = lane; j < nv; j += 8) s = s + sw[j];
    float sum = ((__shfl(s, 0) + __shfl(s, 4)) + (__shfl(s, 1) + __shfl(s, 5))) +
                ((__shfl(s, 2) + __shfl(s, 6)) + (__shfl(s, 3) + __shfl(s, 7)));
    for (int64_t j = nv; j < n; j++) sum = sum + sw[j];
    int64_t nmax = 0;
    int first = -1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        nmax = ns[i] > nmax ? ns[i] : nmax;
        if (first < 0 && ns[i] > 0) first = i;
    }
    bool same = true;
#pragma unroll
    for (int i = 0; i < 4; i++) same = same && (ns[i] == 0 || k0s[i] == k0s[first < 0 ? 0 : first]);
    constexpr int VC = attq_vc<F16>(), VS = attq_vs<F16>();
    constexpr int PPB = F16 ? 1 : 2;  // 16-byte pieces per (dim, 8-key block)
    const int hk = h / (H / Hkv);
    float acc = 0.f;
    for (int pass = 0; pass < (same ? 1 : 4); pass++) {
        const int src = same ? (first < 0 ? 0 : first) : pass;
        const int64_t pn = same ? nmax : ns[pass];
        const bool mine = same || pass == w;
        for (int64_t c0 = 0; c0 < pn; c0 += VC) {
            const int64_t rows = pn - c0 < VC ? pn - c0 : VC;
            // the chunk's keys k0 + c0 .. + rows - 1, dim-major from the block
            // holding the first: key k0 + c0 + j of dim d0 + l at
            // vb[l * VS + offc + j]
            const int64_t ka = k0s[src] + c0, kaa = ka & ~(int64_t)7, offc = ka - kaa;
            const int64_t nblk = (offc + rows + 7) >> 3;
            const VT* vsrc = (const VT*)vc + vcache_at(hk, kaa, d0, D, C);
            __syncthreads();  // the previous chunk has been used
            const int64_t npc = nblk * 64 * PPB;
            for (int64_t i0 = tid; i0 < npc; i0 += 4 * 256) {  // four loads a lane in flight
                uint4 raw[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int64_t i = i0 + 256 * u < npc ? i0 + 256 * u : npc - 1;
                    const int64_t jb = i / (64 * PPB);
                    const int rem = (int)(i - jb * (64 * PPB)), dl = rem / PPB, pc = rem - dl * PPB;
                    raw[u] = *(const uint4*)(vsrc + (jb * D + dl) * 8 + pc * 4);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int64_t i = i0 + 256 * u;
                    if (i < npc) {
                        const int64_t jb = i / (64 * PPB);
                        const int rem = (int)(i - jb * (64 * PPB)), dl = rem / PPB, pc = rem - dl * PPB;
                        *(uint4*)(vb + dl * VS + 8 * jb + pc * 4) = raw[u];
                    }
                }
            }
            __syncthreads();
            if (mine && !bad && c0 < n) {
                const int64_t e1 = n - c0 < rows ? n - c0 : rows;
                const float* e = sw + c0;
                const VT* vd = vb + lane * VS + offc;
                // one key at a time up to a block boundary, then eight keys
                // per read (16-byte aligned: VS and the block starts are)
                int64_t j = 0;
                for (; j < e1 && ((offc + j) & 7); j++) acc = __builtin_fmaf(e[j], (float)vd[j], acc);
                for (; j + 8 <= e1; j += 8) {
                    const uint4 v0 = *(const uint4*)(vd + j);
                    uint4 v1 = v0;
                    if constexpr (!F16) v1 = *(const uint4*)(vd + j + 4);
                    float ev[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) ev[k] = e[j + k];
                    float4 ea = {ev[0], ev[1], ev[2], ev[3]}, eb = {ev[4], ev[5], ev[6], ev[7]};
                    float et[8];
                    *(float4*)et = ea;
                    *(float4*)(et + 4) = eb;
                    att_chain8<F16>(acc, et, v0, v1);
                }
                for (; j < e1; j++) acc = __builtin_fmaf(e[j], (float)vd[j], acc);
            }
        }
    }
    if (t < T) out[((int64_t)t * H + h) * D + d0 + lane] = n <= 0 ? 0.f : (bad ? __builtin_nanf("") : acc / sum);
}

// The weighted sum for few queries (decode), a workgroup of four waves per
// (64 dims d0.., head h, query t). The wave that runs the serial chains
// (wave 0) issues as little else as it can: a dependent fma takes about 10
// cycles on MI355X and every other instruction of that wave adds about 4;
// the others feed it:
//   1. waves 1 and 2 copy the dims' value blocks (8 keys x 64 dims, 1 KB in
//      f16) into a ring of NR batches of 16 blocks in LDS with
//      global_load_lds, NR - 1 batches ahead, starting before anything else
//      (alternate blocks in f16, one 16-byte piece each of every block in
//      f32: one wave issues such a copy only about every 60-100 cycles);
//   2. waves 0 and 3: the scores of the visible keys to LDS (eight loads a
//      lane in flight), max, NaN check; all waves: e = Cephes exp(s - max)
//      for the first n&~7 keys (four a lane) and, on wave 3's last lanes,
//      the f64 exp for the rest, at e[off + j] for key k0 + j (off = k0 % 8:
//      the value blocks start at k0 - off);
//   3. per batch, after a workgroup barrier (the copying waves wait for the
//      batch's copies first), wave 0 lane l runs acc = fma(e_j, v_j[d0+l],
//      acc) over the batch's keys in order (keys outside k0..k0+n-1 of the
//      first and last block skipped, one at a time), and the copying waves
//      start the batch NR - 1 ahead in the slot wave 0 has finished;
//   4. wave 3's lanes 0..7 (during the first batch) sum e over the keys
//      j < n&~7 with j = c mod 8, in order; the sum is ((s0+s4)+(s1+s5))+((s2+s6)+(s3+s7)) plus the rest
//      in order; o[d] = acc / sum.
// The float steps and their order are those of the reference's attendRow
// (attn_amd64.s): the chain per dim in key order, the eight-lane exp sum.

// Global -> LDS copy of 16 bytes a lane (lane i writes at the wave's LDS
// base + 16i), written as inline assembly so that the compiler does not
// count it: the copying waves' waits are explicit (ATT_WAIT_VMCNT).
__device__ __forceinline__ void att_lds_copy16(const void* g, const void* lds_wave_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_wave_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
// s_waitcnt with vmcnt <= n (n < 64), the other counters unconstrained.
#define ATT_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

__device__ __forceinline__ void att_barrier() {  // s_barrier without __syncthreads' vmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads and writes done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}


template <bool F16>
constexpr int att_bb() {  // blocks of 8 keys per batch
    return 16;
}
template <bool F16>
constexpr int att_nr() {  // ring batches: NR - 1 in flight, at most 48 copies a copying wave (vmcnt <= 63)
    return F16 ? 4 : 3;
}
template <bool F16>
constexpr int att_batch_bytes() {
    return att_bb<F16>() * (F16 ? 1 : 2) * 1024;
}

template <bool F16>
__global__ __launch_bounds__(256) void att_wsum_kernel(const void* vc, const int64_t* __restrict__ kend,
                                                       const int64_t* __restrict__ kstart, int H, int Hkv, int D,
                                                       int64_t C, int64_t maxk, const float* __restrict__ ws,
                                                       float* __restrict__ out) {
    constexpr int PPB = F16 ? 1 : 2, BB = att_bb<F16>(), NR = att_nr<F16>(), BATCH = att_batch_bytes<F16>();
    extern __shared__ __align__(16) uint8_t att_lds8[];
    uint8_t* ring = att_lds8;                   // [NR][BB][PPB][64 lanes][16 bytes]
    float* e = (float*)(att_lds8 + NR * BATCH);  // e[off + j]
    __shared__ float red[4];
    __shared__ float lsum[8];
    __shared__ int nan_any;
    const int d0 = 64 * blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const AttRange r = att_range(kend, kstart, t, C, maxk);
    const int64_t n = r.n;
    float* orow = out + ((int64_t)t * H + h) * D + d0;
    const int d = d0 + lane;
    if (n <= 0) {
        if (w == 0 && d < D) orow[lane] = 0.f;
        return;
    }
    const int64_t k0a = r.k0 & ~(int64_t)7;
    const int off = (int)(r.k0 - k0a), nb = (int)((off + n + 7) >> 3), nbat = (nb + BB - 1) / BB;
    // 1. the copying waves (1 and 2: alternate blocks in f16, a 16-byte
    // piece each of every block in f32; one wave issues such a copy about
    // every 96 cycles, slower than the chain takes a block) start the ring
    // (dims past D copy dim D - 1, unused)
    const bool copier = w == 1 || w == 2;
    const int cw = w - 1;
    constexpr int CPB = F16 ? BB / 2 : BB;  // copies a batch a copying wave
    const int hk = h / (H / Hkv);
    using VT = typename std::conditional<F16, _Float16, float>::type;
    const VT* vsrc = (const VT*)vc + vcache_at(hk, k0a, d < D ? d : D - 1, D, C) + (F16 ? 0 : 4 * cw);
    const int64_t bstride = (int64_t)8 * D;
    auto issue_batch = [&](int k) {  // blocks past the last: the last block again
        uint8_t* slot = ring + (k % NR) * BATCH + (F16 ? 0 : cw * 1024);
#pragma unroll
        for (int ii = 0; ii < CPB; ii++) {
            const int i = F16 ? 2 * ii + cw : ii;
            const int b = BB * k + i < nb ? BB * k + i : nb - 1;
            att_lds_copy16(vsrc + b * bstride, slot + i * PPB * 1024);
        }
    };
    if (copier)
        for (int k = 0; k < NR - 1; k++) issue_batch(k);
    // 2. scores (waves 0 and 3), max, NaN check, exps
    // (the copying waves load no scores: the compiler's wait for such loads
    // would also wait for their copies issued before. Eight loads a lane in
    // flight, past the end the last score again, which leaves the max and
    // the NaN check as they are.)
    if (tid == 0) nan_any = 0;
    float mx = -INFINITY;
    int isnan_local = 0;
    if (!copier) {
        const float* srow = ws + ((int64_t)t * H + h) * maxk;
        const int li = w == 0 ? lane : 64 + lane, nl = 128;
        for (int64_t j0 = li; j0 < n; j0 += 8 * nl) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int64_t j = j0 + (int64_t)u * nl;
                v[u] = srow[j < n ? j : n - 1];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int64_t j = j0 + (int64_t)u * nl;
                isnan_local |= v[u] != v[u];
                mx = fmaxf(mx, v[u]);
                if (j < n) e[off + j] = v[u];
            }
        }
    }
    att_barrier();  // nan_any cleared before it is set
    mx = wave_max_f32(mx);
    if (lane == 0) red[w] = mx;
    if (isnan_local) nan_any = 1;
    att_barrier();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool bad = nan_any || __builtin_isinf(mx);
    const int64_t nv = n >= 8 ? (n & ~(int64_t)7) : 0;
    if (!bad) {
        for (int64_t j0 = tid; j0 < nv; j0 += 1024) {  // four a lane, every read first
            float x[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int64_t j = j0 + 256 * u;
                x[u] = e[off + (j < nv ? j : nv - 1)] - mx;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) x[u] = cephes_exp(x[u]);
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (j0 + 256 * u < nv) e[off + j0 + 256 * u] = x[u];
        }
        const int tj = tid - (256 - (int)(n - nv));  // the last n % 8 on wave 3's last lanes
        if (tj >= 0) e[off + nv + tj] = (float)exp((double)(e[off + nv + tj] - mx));
    }
    if (bad) {
        if (w == 0 && d < D) orow[lane] = __builtin_nanf("");
        if (copier) ATT_WAIT_VMCNT(0);  // the ring's copies land before the workgroup's LDS is released
        return;
    }
    att_barrier();  // the exps are written
    // 3. the batches
    float acc = 0.f;
    const int iend = off + (int)n;
    for (int k = 0; k < nbat; k++) {
        if (copier) ATT_WAIT_VMCNT(CPB * (NR - 2));  // batch k has landed
        att_barrier();
        if (k == 0 && w == 3 && lane < 8) {  // 4. the lane sums, beside the first batch's chain
            float sl = 0.f;
            int64_t j = lane;
            for (; j + 120 < nv; j += 128) {
                float ev[16];
#pragma unroll
                for (int u = 0; u < 16; u++) ev[u] = e[off + j + 8 * u];
#pragma unroll
                for (int u = 0; u < 16; u++) sl = sl + ev[u];
            }
            for (; j < nv; j += 8) sl = sl + e[off + j];
            lsum[lane] = sl;
        }
        if (w == 0) {
            const uint8_t* slot = ring + (k % NR) * BATCH + 16 * lane;
            const int b0 = BB * k;
            if (8 * b0 >= off && 8 * (b0 + BB) <= iend) {
                // a batch of whole blocks, straight-line: every value read
                // issued first, the exps as the chain goes (LDS latency is
                // paid once a batch, not once a block)
                uint4 v0[BB], v1[BB];
#pragma unroll
                for (int i = 0; i < BB; i++) {
                    v0[i] = *(const uint4*)(slot + i * PPB * 1024);
                    v1[i] = v0[i];
                    if constexpr (!F16) v1[i] = *(const uint4*)(slot + i * PPB * 1024 + 1024);
                }
                const float* eb = e + 8 * b0;
                float4 ex[2 * BB];
#pragma unroll
                for (int i = 0; i < 2 * BB; i++) ex[i] = *(const float4*)(eb + 4 * i);
                __builtin_amdgcn_sched_barrier(0);  // every read issued before the chain
#pragma unroll
                for (int i = 0; i < BB; i++) {
                    float ev[8];
                    ev[0] = ex[2 * i].x, ev[1] = ex[2 * i].y, ev[2] = ex[2 * i].z, ev[3] = ex[2 * i].w;
                    ev[4] = ex[2 * i + 1].x, ev[5] = ex[2 * i + 1].y, ev[6] = ex[2 * i + 1].z, ev[7] = ex[2 * i + 1].w;
                    att_chain8<F16>(acc, ev, v0[i], v1[i]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < BB; i++) {
                    const int b = BB * k + i;
                    if (b >= nb) break;  // uniform
                    const uint4 v0 = *(const uint4*)(slot + i * PPB * 1024);
                    uint4 v1 = v0;
                    if constexpr (!F16) v1 = *(const uint4*)(slot + i * PPB * 1024 + 1024);
                    const int i0 = 8 * b;
                    if (i0 >= off && i0 + 8 <= iend) {
                        float ev[8];
                        const float4 ea = *(const float4*)(e + i0), eb = *(const float4*)(e + i0 + 4);
                        ev[0] = ea.x, ev[1] = ea.y, ev[2] = ea.z, ev[3] = ea.w;
                        ev[4] = eb.x, ev[5] = eb.y, ev[6] = eb.z, ev[7] = eb.w;
                        att_chain8<F16>(acc, ev, v0, v1);
                    } else {  // the first or last block, partly visible: one key at a time
                        const int lo = i0 > off ? i0 : off, hi = i0 + 8 < iend ? i0 + 8 : iend;
                        for (int ii = lo; ii < hi; ii++) acc = __builtin_fmaf(e[ii], att_vget<F16>(v0, v1, ii - i0), acc);
                    }
                }
            }
        }
        if (copier) issue_batch(k + NR - 1);  // the slot of batch k - 1, which wave 0 has finished
    }
    if (copier) ATT_WAIT_VMCNT(0);  // the ring's last copies (never read) land before the workgroup ends
    att_barrier();  // the lane sums
    if (w == 0 && d < D) {
        float sum = ((lsum[0] + lsum[4]) + (lsum[1] + lsum[5])) + ((lsum[2] + lsum[6]) + (lsum[3] + lsum[7]));
        for (int64_t j = nv; j < n; j++) sum = sum + e[off + j];
        orow[lane] = acc / sum;
    }
}

static void launch_att_wsum(int T, int H, int Hkv, int D, int64_t C, int64_t maxk, int f16, const void* vc,
                            const int64_t* kend, const int64_t* kstart, const float* ws, float* out, hipStream_t s) {
    const size_t e_bytes = (size_t)(((maxk + 7 + 7) & ~(int64_t)7) * 4);
    const dim3 grid((unsigned)((D + 63) / 64), (unsigned)H, (unsigned)T);
    if (f16)
        hipLaunchKernelGGL(att_wsum_kernel<true>, grid, dim3(256), att_nr<true>() * att_batch_bytes<true>() + e_bytes, s,
                           vc, kend, kstart, H, Hkv, D, C, maxk, ws, out);
    else
        hipLaunchKernelGGL(att_wsum_kernel<false>, grid, dim3(256), att_nr<false>() * att_batch_bytes<false>() + e_bytes,
                           s, vc, kend, kstart, H, Hkv, D, C, maxk, ws, out);
}

// swiglu.v1 (reference interp/fast.go:487-498): the reference splits the n
// elements into pieces of `chunk` (parallel(), interp/pool.go:33-51, 79-97)
// and runs SiluMulF32 (attn.go:63-76) on each: the first len&~7 elements of
// a piece through the vector formula, the rest as
// f32(f64(g)/(1+exp(-f64(g)))*f64(u)).
__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out, int64_t n,
                              int64_t chunk) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = swiglu_at(g[i], u[i], i, n, chunk);
}

// One 1024-thread workgroup per row of logits: the first index of the max.
// Each thread scans its elements in increasing index order (eight 16-byte
// loads in flight when the row is 16-byte aligned), keeping the first index
// of its largest value; the group then reduces lexicographically (larger
// value, then smaller index). As the reference's loop (best = 0; x >
// v[best]): NaNs are never chosen, and a row whose first value is NaN gives 0.
__device__ __forceinline__ void am_take(float v, int i, float& best, int& idx, int none) {
    if (idx == none ? v == v : v > best) {
        best = v;
        idx = i;
    }
}
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t n, int32_t* __restrict__ out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float* r = x + (int64_t)blockIdx.x * n;
    const int none = (int)n;
    float best = -INFINITY;
    int idx = none;
    const int tid = threadIdx.x;
    int i0 = 0;
    if (((uintptr_t)r & 15) == 0) {
        // thread tid takes the float4s tid, tid+1024, ... in order: its
        // indices increase, so its first maximum is kept
        const int n4 = (int)(n / 4);
        for (int b = 0; b < n4; b += 8 * 1024) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = b + k * 1024 + tid;
                v[k] = i < n4 ? ((const float4*)r)[i] : make_float4(NAN, NAN, NAN, NAN);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = 4 * (b + k * 1024 + tid);
                am_take(v[k].x, i, best, idx, none);
                am_take(v[k].y, i + 1, best, idx, none);
                am_take(v[k].z, i + 2, best, idx, none);
                am_take(v[k].w, i + 3, best, idx, none);
            }
        }
        i0 = n4 * 4;
    }
    for (int i = i0 + tid; i < (int)n; i += 1024) am_take(r[i], i, best, idx, none);
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(idx, off);
        if (oi != none && (idx == none || ov > best || (ov == best && oi < idx))) {
            best = ov;
            idx = oi;
        }
    }
    const int w = tid >> 6;
    if ((tid & 63) == 0) {
        bv[w] = best;
        bi[w] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        int i0b = bi[0];
        for (int k = 1; k < 16; k++)
            if (bi[k] != none && (i0b == none || bv[k] > b || (bv[k] == b && bi[k] < i0b))) {
                b = bv[k];
                i0b = bi[k];
            }
        // the reference starts from index 0, which no NaN-led row leaves
        out[blockIdx.x] = (int32_t)(i0b == none || r[0] != r[0] ? 0 : i0b);
    }
}

// One step of the greedy loop on the device (reference cmd/mim-run/main.go
// generate): the chosen token becomes the next input, is appended to out
// (while count < cap), and the position and cache index advance by one.
__global__ void greedy_advance_kernel(const int32_t* __restrict__ chosen, int32_t* __restrict__ ids,
                                      int64_t* __restrict__ pos, int64_t* __restrict__ cidx, int32_t* __restrict__ out,
                                      int32_t* __restrict__ count, int cap, int n) {
    const int i = threadIdx.x;
    const int c = count[0];
    if (i < n) {
        ids[i] = chosen[i];
        if (c >= 0 && c < cap) out[(int64_t)c * n + i] = chosen[i];
        pos[i] += 1;
        if (cidx) cidx[i] += 1;
    }
    __syncthreads();
    if (i == 0) count[0] += 1;
}

hipError_t launch_greedy_advance(const int32_t* chosen, int32_t* ids, int64_t* pos, int64_t* cidx, int32_t* out,
                                 int32_t* count, int cap, int n, hipStream_t s) {
    if (n < 1 || n > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(greedy_advance_kernel, dim3(1), dim3(1024), 0, s, chosen, ids, pos, cidx, out, count, cap, n);
    return hipGetLastError();
}

hipError_t launch_embed_rows(uint32_t dt, const uint8_t* table, int64_t row_bytes, const int32_t* ids, int T, int V,
                             int64_t E, float* out, hipStream_t s) {
    dim3 grid((unsigned)((E + 255) / 256), (unsigned)T);
    switch (dt) {
    case DT_Q4_K: hipLaunchKernelGGL(embed_rows_kernel<DT_Q4_K>, grid, dim3(256), 0, s, table, row_bytes, ids, V, E, out); break;
    case DT_Q6_K: hipLaunchKernelGGL(embed_rows_kernel<DT_Q6_K>, grid, dim3(256), 0, s, table, row_bytes, ids, V, E, out); break;
    case DT_Q8_0: hipLaunchKernelGGL(embed_rows_kernel<DT_Q8_0>, grid, dim3(256), 0, s, table, row_bytes, ids, V, E, out); break;
    case DT_F32: hipLaunchKernelGGL(embed_rows_kernel<DT_F32>, grid, dim3(256), 0, s, table, row_bytes, ids, V, E, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rms_norm(float* x, const float* resid, const float* scale, float eps, int64_t rows, int64_t n, float* y,
                           hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, resid, scale, eps, n, y);
    return hipGetLastError();
}

hipError_t launch_rope(float* x, const int64_t* pos, const double* inv_freq, int T, int heads, int D, int rotary,
                       int interleaved, hipStream_t s) {
    const int64_t total = (int64_t)T * heads * (rotary / 2);
    const unsigned grid = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(rope_kernel, dim3(grid ? grid : 1), dim3(256), 0, s, x, pos, inv_freq, T, heads, D, rotary,
                       interleaved);
    return hipGetLastError();
}

hipError_t launch_kv_store(const float* k, const float* v, const int64_t* pos, int T, int Hkv, int D, int64_t C, void* kc,
                           void* vc, int f16, hipStream_t s) {
    const int64_t total = (int64_t)T * Hkv * D;
    const unsigned grid = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(kv_store_kernel, dim3(grid ? grid : 1), dim3(256), 0, s, k, v, pos, T, Hkv, D, C, kc, vc, f16);
    return hipGetLastError();
}

// Prompt scores with a key per lane (many queries over one sequence): a
// workgroup per (tiles of 256 cache entries, head, QG queries): the tiles
// from the first entry any of its queries sees, blockIdx.x, gridDim.x
// apart; thread i holds the key of cache entry kb + i (D values, f16 or
// f32, in registers) and the QG query rows sit in LDS, read as broadcasts. For each query the lane runs
// the reference's eight chains itself, l_c = fma(q[8m + c], k[8m + c], l_c)
// for m = 0..D/8-1 in order, and combines them with the pairing
// att_reduce8 uses (((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)) for keys in the
// groups of four, ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) for the last n % 4):
// the same operations on the same values as att_scores_kernel, so the same
// bits, without its eight-lane split (sixteen 2-byte loads and a DPP
// reduction per key and query). A wave skips a query none of its 64 keys is
// visible to; stores are consecutive keys.
// A value every lane holds the same copy of (read from LDS), made a scalar
// so that comparisons on it are scalar branches, not exec masks.
__device__ __forceinline__ int64_t uni64(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

constexpr int ATT_KPL_QG = 32;

template <bool F16, int D>
__global__ __launch_bounds__(256) void att_scores_kpl_kernel(const float* __restrict__ q, const void* kc,
                                                             const int64_t* __restrict__ kend,
                                                             const int64_t* __restrict__ kstart, int T, int H,
                                                             int Hkv, int64_t C, int64_t maxk,
                                                             float* __restrict__ ws) {
    constexpr int QG = ATT_KPL_QG, DM = D / 8;
    constexpr int KW = F16 ? D / 2 : D;  // 32-bit words of a key
    __shared__ __align__(16) float qs[QG * D];
    __shared__ int64_t k0s[QG], ns[QG];
    const int h = blockIdx.y, tid = threadIdx.x, w = tid >> 6;
    const int hk = h / (H / Hkv), t0 = (int)blockIdx.z * QG;
    if (tid < QG) {
        const int t = t0 + tid;
        const AttRange r = t < T ? att_range(kend, kstart, t, C, maxk) : AttRange{0, 0};
        k0s[tid] = r.k0;
        ns[tid] = r.n;
    }
    __syncthreads();
    // the cache entries the queries see: [kmin, kfin); this workgroup takes
    // the tiles of 256 of them from tile blockIdx.x, gridDim.x apart
    int64_t kmin = INT64_MAX, kfin = 0;
#pragma unroll
    for (int i = 0; i < QG; i++) {
        const int64_t ni = uni64(ns[i]), ki = uni64(k0s[i]);
        if (ni <= 0) continue;
        kmin = ki < kmin ? ki : kmin;
        kfin = ki + ni > kfin ? ki + ni : kfin;
    }
    if (kfin == 0) return;  // uniform: no query sees a key
    // the query rows (zeros past T: never stored)
    for (int i = tid; i < QG * D / 4; i += 256) {
        const int tq = i / (D / 4), d4 = i - tq * (D / 4), t = t0 + tq;
        const float4 v = t < T ? *(const float4*)(q + ((int64_t)t * H + h) * D + 4 * d4) : float4{0.f, 0.f, 0.f, 0.f};
        *(float4*)(qs + tq * D + 4 * d4) = v;
    }
    __syncthreads();
    for (int64_t kb = kmin + 256 * (int64_t)blockIdx.x; kb < kfin; kb += 256 * (int64_t)gridDim.x) {
    // this lane's key (entries past the cache read the last one, unstored)
    const int64_t a = kb + tid, ac = a < C ? a : C - 1;
    uint32_t kw[KW];
    {
        const uint4* kp = (const uint4*)((const uint8_t*)kc + ((int64_t)hk * C + ac) * D * (F16 ? 2 : 4));
#pragma unroll
        for (int i = 0; i < KW / 4; i++) {
            const uint4 v = kp[i];
            kw[4 * i] = v.x;
            kw[4 * i + 1] = v.y;
            kw[4 * i + 2] = v.z;
            kw[4 * i + 3] = v.w;
        }
    }
    const float scale = (float)(1.0 / sqrt((double)D));
    const int64_t wa = kb + 64 * w;  // this wave's first cache entry
    for (int i = 0; i < QG; i++) {
        const int64_t k0 = uni64(k0s[i]), n = uni64(ns[i]);
        if (n <= 0 || k0 >= wa + 64 || k0 + n <= wa) continue;  // uniform
        const float* qr = qs + i * D;
        float l[8];
#pragma unroll
        for (int c = 0; c < 8; c++) l[c] = 0.f;
#pragma unroll
        for (int m = 0; m < DM; m++) {
            const float4 qa = *(const float4*)(qr + 8 * m), qb = *(const float4*)(qr + 8 * m + 4);
            const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int c = 0; c < 8; c++) {
                float kv;
                if constexpr (F16) {
                    const uint32_t wd = kw[4 * m + c / 2];
                    kv = (float)__builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? wd >> 16 : wd & 0xFFFF));
                } else {
                    kv = __uint_as_float(kw[8 * m + c]);
                }
                l[c] = __builtin_fmaf(qv[c], kv, l[c]);
            }
        }
        const int64_t j = a - k0, n4 = n - n % 4;
        const float pf = ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
        const float pn = ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
        const float p = j < n4 ? pf : pn;
        if (j >= 0 && j < n) ws[((int64_t)(t0 + i) * H + h) * maxk + j] = p * scale;
    }
    }
}

// Prompt weighted sum with queries' chains side by side: a workgroup per
// (head, QG queries) of D/64 x QG/QW waves; a wave takes 64 dims of the head
// and QW of the queries, each lane the QW chains acc_q = fma(e_q[j],
// v_j[d], acc_q) of its dim in key order (the same chains as
// att_wsum_q4_kernel, which gives a wave one query: here QW independent
// fmas follow each value, so the chains' latency is hidden). The value of
// key j is read straight from the blocked cache (one 16-byte load gives
// eight keys of the dim), four blocks ahead; a block's weights are read
// from LDS before its fmas. Per query first: max and NaN check over its
// scores, e = Cephes exp(s - max) for the first n & ~7 keys and the f64 exp
// for the rest, into LDS as [key][query]; the eight stride-8 lane sums in
// key order, ((s0+s4)+(s1+s5))+((s2+s6)+(s3+s7)) and the rest in order;
// o[d] = acc / sum (NaN for a NaN score or an infinite max, 0 for no
// visible key). Queries that do not share the first visible entry run in
// passes of one.
constexpr int ATT_QPL_QG = 16, ATT_QPL_QW = 8;

template <bool F16, int D>
__global__ __launch_bounds__(D * ATT_QPL_QG / ATT_QPL_QW) void att_wsum_qpl_kernel(
    const void* vc, const int64_t* __restrict__ kend, const int64_t* __restrict__ kstart, int T, int H, int Hkv,
    int64_t C, int64_t maxk, const float* __restrict__ ws, float* __restrict__ out) {
    constexpr int QG = ATT_QPL_QG, QW = ATT_QPL_QW, DH = D / 64, NT = D * QG / QW, NWV = NT / 64;
    using VT = typename std::conditional<F16, _Float16, float>::type;
    extern __shared__ __align__(16) float ew[];  // [maxk][QG]
    __shared__ int64_t k0s[QG], ns[QG];
    __shared__ float sums[QG];
    __shared__ int bads[QG];
    __shared__ float mxs[NWV][QG];
    __shared__ int bws[NWV][QG];
    const int h = blockIdx.y, t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int d = lane + 64 * (w % DH), qg = w / DH;  // this lane's dim and query group
    const int hk = h / (H / Hkv), t0 = (int)blockIdx.z * QG;
    if (t < QG) {
        const int tq = t0 + t;
        const AttRange r = tq < T ? att_range(kend, kstart, tq, C, maxk) : AttRange{0, 0};
        k0s[t] = r.k0;
        ns[t] = r.n;
    }
    __syncthreads();
    // 1. Every query's scores into LDS ([key][query]), eight loads a thread
    // in flight (the index space is QG rows of a power-of-two length, so a
    // row and a key are a shift and a mask); then max, NaN check and the
    // exps in place, thread t on query t % QG and keys t / QG + k NT / QG (so
    // consecutive threads touch consecutive words), the maxima and the NaN
    // flags combined across the threads of a query.
    int64_t nall = 0;
#pragma unroll
    for (int i = 0; i < QG; i++) nall = ns[i] > nall ? ns[i] : nall;
    int lg = 0;
    while ((1ll << lg) < nall) lg++;
    const int64_t span = (int64_t)QG << lg;
    for (int64_t b0 = t; b0 < (nall > 0 ? span : 0); b0 += 8 * NT) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t idx = b0 + (int64_t)NT * u;
            const int qi = (int)(idx >> lg) & (QG - 1);
            const int64_t j = idx & ((1ll << lg) - 1);
            const bool ok = idx < span && j < ns[qi];
            v[u] = ok ? ws[((int64_t)(t0 + qi) * H + h) * maxk + j] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t idx = b0 + (int64_t)NT * u;
            const int qi = (int)(idx >> lg) & (QG - 1);
            const int64_t j = idx & ((1ll << lg) - 1);
            if (idx < span && j < ns[qi]) ew[j * QG + qi] = v[u];
        }
    }
    __syncthreads();
    {
        constexpr int JS = NT / QG;  // keys a step
        const int qi = t & (QG - 1), jj = t / QG;
        const int64_t n = ns[qi];
        float mx = -INFINITY;
        int bad = 0;
        for (int64_t j = jj; j < n; j += JS) {
            const float v = ew[j * QG + qi];
            bad |= v != v;
            mx = fmaxf(mx, v);
        }
        // the threads of query qi: lanes qi + 16m of each wave, then the waves
        mx = fmaxf(mx, lane_xor_f32<16>(mx));
        mx = fmaxf(mx, lane_xor_f32<32>(mx));
        bad |= __shfl_xor(bad, 16);
        bad |= __shfl_xor(bad, 32);
        if (lane < QG) {
            mxs[w][lane] = mx;
            bws[w][lane] = bad;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NWV; i++) {
            mx = fmaxf(mx, mxs[i][qi]);
            bad |= bws[i][qi];
        }
        bad = bad || __builtin_isinf(mx);
        const int64_t nv = n >= 8 ? (n & ~(int64_t)7) : 0;
        if (!bad)
            for (int64_t j = jj; j < n; j += JS) {
                const float x = ew[j * QG + qi] - mx;
                ew[j * QG + qi] = j < nv ? cephes_exp(x) : (float)exp((double)x);
            }
        if (t < QG) bads[t] = bad;
    }
    __syncthreads();
    // 2. The sums: thread 8i + c (i < QG) runs query i's chain c.
    if (t < 8 * QG) {
        const int qi = t >> 3, c = t & 7;
        const int64_t n = ns[qi], nv = n >= 8 ? (n & ~(int64_t)7) : 0;
        float sl = 0.f;
        for (int64_t j = c; j < nv; j += 8) sl = sl + ew[j * QG + qi];
        const int g = lane & ~7;
        float sum = ((__shfl(sl, g) + __shfl(sl, g + 4)) + (__shfl(sl, g + 1) + __shfl(sl, g + 5))) +
                    ((__shfl(sl, g + 2) + __shfl(sl, g + 6)) + (__shfl(sl, g + 3) + __shfl(sl, g + 7)));
        if (c == 0) {
            for (int64_t j = nv; j < n; j++) sum = sum + ew[j * QG + qi];
            sums[qi] = sum;
        }
    }
    __syncthreads();
    // 3. The chains of this wave's queries, in passes of the workgroup's
    // queries that share the first entry. Keys below every live query's
    // count run unmasked, whole value blocks at a time; the rest key by key
    // with each query's own bound. Every bound is a scalar.
    const int q0 = QW * qg;
    float acc[QW];
#pragma unroll
    for (int i = 0; i < QW; i++) acc[i] = 0.f;
    int64_t nq[QW];
    int bq[QW];
#pragma unroll
    for (int i = 0; i < QW; i++) {
        nq[i] = uni64(ns[q0 + i]);
        bq[i] = __builtin_amdgcn_readfirstlane(bads[q0 + i]);
    }
    int first = -1;
    bool same = true;
    for (int i = 0; i < QG; i++) {
        const int64_t ni = uni64(ns[i]);
        if (ni <= 0) continue;
        if (first < 0) first = i;
        else same = same && uni64(k0s[i]) == uni64(k0s[first]);
    }
    const VT* vbase = (const VT*)vc;
    for (int pass = 0; pass < (same ? 1 : QG); pass++) {
        if (!same && (pass < q0 || pass >= q0 + QW)) continue;  // not this wave's query
        const int src = same ? (first < 0 ? 0 : first) : pass;
        if (uni64(ns[src]) <= 0) continue;
        const int64_t k0 = uni64(k0s[src]);
        uint32_t live = 0;
        int64_t nmin = INT64_MAX, nmax = 0;
#pragma unroll
        for (int i = 0; i < QW; i++) {
            const bool in = nq[i] > 0 && !bq[i] && (same || q0 + i == pass);
            if (in) {
                live |= 1u << i;
                nmin = nq[i] < nmin ? nq[i] : nmin;
                nmax = nq[i] > nmax ? nq[i] : nmax;
            }
        }
        if (!live) continue;
        const int64_t nfull = live == (1u << QW) - 1 ? nmin : 0;  // keys every query of the wave sees
        const int64_t off = k0 & 7;                                 // key k0's place in its value block
        const int64_t kbeg = k0 - off;
        const int64_t nblk = (off + nmax + 7) >> 3;
        auto vload = [&](int64_t ib, uint4& x0, uint4& x1) {
            const VT* vp = vbase + vcache_at(hk, kbeg + 8 * (ib < nblk ? ib : nblk - 1), d, D, C);
            x0 = *(const uint4*)vp;
            x1 = x0;
            if constexpr (!F16) x1 = *(const uint4*)(vp + 4);
        };
        constexpr int PF = 4;
        uint4 c0[PF], c1[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) vload(u, c0[u], c1[u]);
        for (int64_t ib0 = 0; ib0 < nblk; ib0 += PF) {
            uint4 n0[PF], n1[PF];
#pragma unroll
            for (int u = 0; u < PF; u++) vload(ib0 + PF + u, n0[u], n1[u]);
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const int64_t ib = ib0 + u;
                if (ib >= nblk) break;
                const int64_t j0 = 8 * ib - off;  // key index of the block's entry 0
                if (j0 >= 0 && j0 + 8 <= nfull) {
                    // a whole block every query sees: its weights first, then the fmas
                    float4 ea[8], eb[8];
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) {
                        const float4* er = (const float4*)(ew + (j0 + kk) * QG + q0);
                        ea[kk] = er[0];
                        eb[kk] = er[1];
                    }
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) {
                        const float v = att_vget<F16>(c0[u], c1[u], kk);
                        const float e[8] = {ea[kk].x, ea[kk].y, ea[kk].z, ea[kk].w,
                                            eb[kk].x, eb[kk].y, eb[kk].z, eb[kk].w};
#pragma unroll
                        for (int i = 0; i < QW; i++) acc[i] = __builtin_fmaf(e[i], v, acc[i]);
                    }
                } else {
                    // the block's keys one at a time, each query to its own count
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) {
                        const int64_t j = j0 + kk;
                        if (j < 0 || j >= nmax) continue;
                        const float4* er = (const float4*)(ew + j * QG + q0);
                        const float4 ea = er[0], eb = er[1];
                        const float e[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
                        const float v = att_vget<F16>(c0[u], c1[u], kk);
#pragma unroll
                        for (int i = 0; i < QW; i++)
                            if (((live >> i) & 1) && j < nq[i]) acc[i] = __builtin_fmaf(e[i], v, acc[i]);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < PF; u++) {
                c0[u] = n0[u];
                c1[u] = n1[u];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < QW; i++) {
        const int qi = q0 + i, tq = t0 + qi;
        if (tq < T)
            out[((int64_t)tq * H + h) * D + d] = ns[qi] <= 0 ? 0.f : (bads[qi] ? __builtin_nanf("") : acc[i] / sums[qi]);
    }
}

template <bool F16, int QT>
static void launch_att_scores(dim3 grid, const float* q, const void* kc, const int64_t* kend, const int64_t* kstart,
                              int T, int H, int Hkv, int D, int64_t C, int64_t maxk, float* ws, hipStream_t s) {
    if (D == 64)
        hipLaunchKernelGGL((att_scores_kernel<F16, 8, QT>), grid, dim3(256), 0, s, q, kc, kend, kstart, T, H, Hkv, D, C,
                           maxk, ws);
    else if (D == 128)
        hipLaunchKernelGGL((att_scores_kernel<F16, 16, QT>), grid, dim3(256), 0, s, q, kc, kend, kstart, T, H, Hkv, D, C,
                           maxk, ws);
    else
        hipLaunchKernelGGL((att_scores_kernel<F16, 0, QT>), grid, dim3(256), 0, s, q, kc, kend, kstart, T, H, Hkv, D, C,
                           maxk, ws);
}


hipError_t launch_attention(const float* q, const void* kc, const void* vc, const int64_t* kend, const int64_t* kstart,
                            int T, int H, int Hkv, int D, int64_t C, int64_t maxk, int f16, float* out, float* ws,
                            hipStream_t s) {
    if (D > 512 || D % 8 || H % Hkv || maxk < 1 || maxk > ATT_MAXC || T < 1) return hipErrorInvalidValue;
    // many queries: four per workgroup, sharing the key and value loads
    const bool many = T >= 16 && D % 64 == 0 && maxk <= 2048;
    const unsigned tiles = (unsigned)((maxk + 63) / 64);
    // many queries, D = 64 or 128 (D = 128 with an f16 cache: the key in 64
    // registers), up to 1024 keys: a key per lane for the scores and the
    // queries' chains side by side for the weighted sum
    // (measured on MI355X at the 8B heads: 125 against 224 us at 512 rows;
    // slower below about 256 rows, whose grids are too small)
    if (many && T >= 256 && (D == 64 || (D == 128 && f16)) && maxk <= 1024 && T <= 65535 &&
        (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15) == 0) {
        const dim3 g1((unsigned)((maxk + 255) / 256), (unsigned)H, (unsigned)((T + ATT_KPL_QG - 1) / ATT_KPL_QG));
        const dim3 g2(1, (unsigned)H, (unsigned)((T + ATT_QPL_QG - 1) / ATT_QPL_QG));
        const size_t lds = (size_t)maxk * ATT_QPL_QG * 4;
#define ATT_PROMPT(F, DD)                                                                                         \
    hipLaunchKernelGGL((att_scores_kpl_kernel<F, DD>), g1, dim3(256), 0, s, q, kc, kend, kstart, T, H, Hkv, C, maxk, \
                       ws);                                                                                       \
    hipLaunchKernelGGL((att_wsum_qpl_kernel<F, DD>), g2, dim3(DD * ATT_QPL_QG / ATT_QPL_QW), lds, s, vc, kend,         \
                       kstart, T, H, Hkv, C, maxk, ws,                                                           \
                       out)
        if (f16 && D == 128) { ATT_PROMPT(true, 128); }
        else if (f16) { ATT_PROMPT(true, 64); }
        else { ATT_PROMPT(false, 64); }
#undef ATT_PROMPT
        return hipGetLastError();
    }
    if (many) {
        const dim3 grid(tiles, (unsigned)H, (unsigned)((T + 3) / 4));
        if (f16) launch_att_scores<true, 4>(grid, q, kc, kend, kstart, T, H, Hkv, D, C, maxk, ws, s);
        else launch_att_scores<false, 4>(grid, q, kc, kend, kstart, T, H, Hkv, D, C, maxk, ws, s);
        const size_t lds = (size_t)(4 * ((maxk + 3) & ~(int64_t)3) * 4 + (f16 ? attq_vs<true>() * 64 * 2 : attq_vs<false>() * 64 * 4));
        const dim3 g2((unsigned)(D / 64), (unsigned)H, (unsigned)((T + 3) / 4));
        if (f16)
            hipLaunchKernelGGL(att_wsum_q4_kernel<true>, g2, dim3(256), lds, s, vc, kend, kstart, T, H, Hkv, D, C, maxk,
                               ws, out);
        else
            hipLaunchKernelGGL(att_wsum_q4_kernel<false>, g2, dim3(256), lds, s, vc, kend, kstart, T, H, Hkv, D, C, maxk,
                               ws, out);
        return hipGetLastError();
    }
    // few queries, D = 64 or 128, at most ATT_DEC_MAXK keys: one launch per
    // query (att_decode_kernel). Its workgroups compute all of a query's
    // scores each, which beats the two-kernel path (scores spread over
    // tiles of 64 keys) only for short contexts (measured on MI355X at
    // D = 128: 4.7 against 7.5 us at 64 keys, 17.9 against 13.6 at 640).
    if ((D == 64 || D == 128) && T <= 65535 && maxk <= ATT_DEC_MAXK) {
        constexpr size_t LDS_MAX = 160 * 1024 - 64;
        const dim3 g((unsigned)(D / 32), (unsigned)H, (unsigned)T);
#define ATT_DEC(F, DD)                                                                                           \
    const size_t lds = att_decode_lds<F, DD>(maxk);                                                              \
    if (lds <= LDS_MAX) {                                                                                        \
        hipLaunchKernelGGL((att_decode_kernel<F, DD, 32>), g, dim3(256), lds, s, q, kc, vc, kend, kstart, H, Hkv, \
                           C, maxk, out);                                                                        \
        return hipGetLastError();                                                                                \
    }
        if (f16 && D == 128) { ATT_DEC(true, 128) }
        else if (f16) { ATT_DEC(true, 64) }
        else if (D == 128) { ATT_DEC(false, 128) }
        else { ATT_DEC(false, 64) }
#undef ATT_DEC
    }
    const int G = H / Hkv;
    // the query heads of a kv head together, each key loaded once, when that
    // grid still gives every CU a workgroup (one query over a short context
    // is faster per head: 4.1 against 4.5 us at 32 heads and 768 keys)
    if ((D == 64 || D == 128) && (G == 2 || G == 4 || G == 8) && !(G == 8 && D == 128) &&
        (long)tiles * Hkv * T >= 256) {
        const dim3 grid(tiles, (unsigned)Hkv, (unsigned)T);
#define ATT_GQA(F, DM, GG) \
    hipLaunchKernelGGL((att_scores_gqa_kernel<F, DM, GG>), grid, dim3(256), 0, s, q, kc, kend, kstart, T, H, Hkv, D, C, maxk, ws)
        if (f16) {
            if (D == 64) { if (G == 2) ATT_GQA(true, 8, 2); else if (G == 4) ATT_GQA(true, 8, 4); else ATT_GQA(true, 8, 8); }
            else { if (G == 2) ATT_GQA(true, 16, 2); else ATT_GQA(true, 16, 4); }
        } else {
            if (D == 64) { if (G == 2) ATT_GQA(false, 8, 2); else if (G == 4) ATT_GQA(false, 8, 4); else ATT_GQA(false, 8, 8); }
            else { if (G == 2) ATT_GQA(false, 16, 2); else ATT_GQA(false, 16, 4); }
        }
#undef ATT_GQA
    } else {
        const dim3 grid(tiles, (unsigned)H, (unsigned)T);
        if (f16) launch_att_scores<true, 1>(grid, q, kc, kend, kstart, T, H, Hkv, D, C, maxk, ws, s);
        else launch_att_scores<false, 1>(grid, q, kc, kend, kstart, T, H, Hkv, D, C, maxk, ws, s);
    }
    launch_att_wsum(T, H, Hkv, D, C, maxk, f16, vc, kend, kstart, ws, out, s);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, const int64_t* pos, const int64_t* cidx,
                          const double* inv_freq, int T, int H, int Hkv, int D, int rotary, int interleaved, int64_t C,
                          void* kc, void* vc, int f16, hipStream_t s) {
    if (D % 2 || D > 1024 || rotary > D || rotary % 2 || (!interleaved && (D - rotary) % 2)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(H + 2 * Hkv), (unsigned)T), blk((unsigned)((D / 2 + 63) / 64 * 64));
    if (f16)
        hipLaunchKernelGGL(rope_kv_kernel<true>, grid, blk, 0, s, q, k, v, pos, cidx, inv_freq, H, Hkv, D, rotary,
                           interleaved, C, kc, vc);
    else
        hipLaunchKernelGGL(rope_kv_kernel<false>, grid, blk, 0, s, q, k, v, pos, cidx, inv_freq, H, Hkv, D, rotary,
                           interleaved, C, kc, vc);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* out, int64_t n, int64_t chunk, hipStream_t s) {
    if (chunk < 1) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid ? grid : 1), dim3(256), 0, s, g, u, out, n, chunk);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int64_t rows, int64_t n, int32_t* out, hipStream_t s) {
    if (n <= 0 || n >= (1ll << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, s, x, n, out);
    return hipGetLastError();
}

}  // namespace mimg
