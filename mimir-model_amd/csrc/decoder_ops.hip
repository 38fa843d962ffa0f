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
#include "f32path.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Rows of the embedding table for the given tokens: out[t][e].
template <uint32_t DT>
__global__ void embed_rows_kernel(const uint8_t* __restrict__ table, int64_t row_bytes, const int32_t* __restrict__ ids,
                                  int V, int64_t E, float* __restrict__ out) {
    const int t = blockIdx.y;
    int id = ids[t];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    const uint8_t* row = table + (int64_t)id * row_bytes;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < E; e += (int64_t)gridDim.x * blockDim.x)
        if constexpr (DT == DT_F32) out[(int64_t)t * E + e] = ((const float*)row)[e];
        else out[(int64_t)t * E + e] = decode_weight<DT>(row, e);
}

// One 256-thread workgroup per row: x += resid (if given, written back to
// x), then y = rms_norm(x) * scale.
__global__ __launch_bounds__(256) void rms_norm_kernel(float* __restrict__ x, const float* __restrict__ resid,
                                                       const float* __restrict__ scale, float eps, int64_t n,
                                                       float* __restrict__ y) {
    __shared__ double part[4];
    __shared__ float inv_s;
    float* xr = x + (int64_t)blockIdx.x * n;
    const float* rr = resid ? resid + (int64_t)blockIdx.x * n : nullptr;
    float* yr = y + (int64_t)blockIdx.x * n;
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        float v = xr[i];
        if (rr) {
            v = v + rr[i];
            xr[i] = v;
        }
        ss += (double)v * (double)v;
    }
    ss = wave_sum_f64(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
        const double tot = (part[0] + part[1]) + (part[2] + part[3]);
        inv_s = (float)(1.0 / sqrt((double)(float)(tot / (double)n) + (double)eps));
    }
    __syncthreads();
    const float inv = inv_s;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i] * inv;
        yr[i] = scale ? v * scale[i] : v;
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

// k, v [T][Hkv][D] into the caches [Hkv][C][D] at the cache indices pos[t]
// (rounded to f16 when the cache is f16).
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
        const int64_t at = ((int64_t)hk * C + p) * D + d;
        if (f16) {
            ((_Float16*)kc)[at] = (_Float16)k[idx];
            ((_Float16*)vc)[at] = (_Float16)v[idx];
        } else {
            ((float*)kc)[at] = k[idx];
            ((float*)vc)[at] = v[idx];
        }
    }
}

__device__ __forceinline__ float kv_at(const void* c, int64_t i, int f16) {
    return f16 ? (float)((const _Float16*)c)[i] : ((const float*)c)[i];
}

// Cephes' expf as the reference's expSumF32AVX2 evaluates it
// (attn_amd64.s:81-240): t clamped to lo, f = rint(t*log2e), r = t - f*ln2
// with ln2 in two parts (fma), exp(r) = 1 + r + r^2 P(r), times 2^f put in
// the exponent; t < lo (and NaN) gives 0.
__device__ __forceinline__ float cephes_exp(float t) {
    const float lo = __uint_as_float(0xc2aeac4fu), log2e = __uint_as_float(0x3fb8aa3bu);
    const float c1 = __uint_as_float(0x3f318000u), c2 = __uint_as_float(0xb95e8083u);
    const bool keep = t >= lo;
    const float tt = t > lo ? t : lo;
    const float f = __builtin_rintf(tt * log2e);
    float r = __builtin_fmaf(-f, c1, tt);
    r = __builtin_fmaf(-f, c2, r);
    const float r2 = r * r;
    float p = __uint_as_float(0x39506967u);
    p = __builtin_fmaf(p, r, __uint_as_float(0x3ab743ceu));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3c088908u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3d2aa9c1u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3e2aaaaau));
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r2, r);
    p = p + 1.0f;
    const float e = p * __uint_as_float((uint32_t)((int32_t)f + 127) << 23);
    return keep ? e : 0.0f;
}

// attention.v1/.v2 for one query row and head, in the reference's attendRow
// order (interp/fast.go:728-751 with attn_amd64.s), so the result is the
// reference's bit for bit. One 256-thread workgroup per (query t, head h)
// over cache entries kstart[t]..kend[t] of kv head h / (H / Hkv), D a
// multiple of 8 (at most 512), at most ATT_MAXC visible keys.
//   scores  eight lanes per key: lane c sums q[8m+c]*k[8m+c] by fma over m;
//           keys go in fours from the first, reduced
//           ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)), the last n%4 keys as
//           ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)); times scale
//   expsum  Cephes exp of s - max for the first n&~7 keys, eight stride-8
//           lane sums in key order, HSUM, then the tail keys with the f64
//           exp added in order
//   wsum    thread d: acc = fma(e_j, v_j[d], acc) over the keys in order;
//           o[d] = acc / sum
// A non-finite largest score gives NaN (the reference's scalar loop ends
// in NaN then); no visible key gives zeros.
constexpr int ATT_MAXC = 8192;
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q, const void* kc, const void* vc,
                                                        const int64_t* __restrict__ kend,
                                                        const int64_t* __restrict__ kstart, int H, int Hkv, int D,
                                                        int64_t C, int f16, float* __restrict__ out) {
    __shared__ float sc[ATT_MAXC];
    __shared__ float qs[512];
    __shared__ float red[4];
    __shared__ int nan_any;
    __shared__ float lane_sum[8];
    const int t = blockIdx.y, h = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int hk = h / (H / Hkv);
    // visible keys, indexed from k0; kept inside the cache row and LDS
    const int64_t k0 = kstart ? (kstart[t] < 0 ? 0 : (kstart[t] >= C ? C - 1 : kstart[t])) : 0;
    int64_t n = kend[t] + 1 - k0;
    if (n > C - k0) n = C - k0;
    if (n > ATT_MAXC) n = ATT_MAXC;
    const int64_t cbase = (int64_t)hk * C + k0;
    const float scale = (float)(1.0 / sqrt((double)D));
    float* orow = out + ((int64_t)t * H + h) * D;
    if (n <= 0) {
        for (int d = tid; d < D; d += 256) orow[d] = 0.f;
        return;
    }
    const float* qr = q + ((int64_t)t * H + h) * D;
    for (int d = tid; d < D; d += 256) qs[d] = qr[d];
    if (tid == 0) nan_any = 0;
    __syncthreads();
    // scores: 32 groups of eight lanes, a key per group
    const int c = lane & 7, gbase = lane & ~7, grp = tid >> 3;
    const int64_t n4 = n - n % 4;
    for (int64_t j0 = 0; j0 < n; j0 += 32) {
        const int64_t j = j0 + grp;
        const int64_t jj = j < n ? j : n - 1;  // groups past the end recompute the last key, unstored
        const int64_t base = (cbase + jj) * D;
        float l = 0.f;
        for (int m = 0; m < D / 8; m++) l = __builtin_fmaf(qs[8 * m + c], kv_at(kc, base + 8 * m + c, f16), l);
        const bool four = jj < n4;
        const int x1 = four ? 1 : 4, x2 = four ? 2 : 1, x3 = four ? 4 : 2;
        float p = l + __shfl(l, gbase + (c ^ x1));
        p = p + __shfl(p, gbase + (c ^ x2));
        p = p + __shfl(p, gbase + (c ^ x3));
        if (c == 0 && j < n) sc[j] = p * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    int isnan_local = 0;
    for (int64_t j = tid; j < n; j += 256) {
        const float v = sc[j];
        isnan_local |= v != v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[w] = mx;
    if (isnan_local) nan_any = 1;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (nan_any || __builtin_isinf(mx)) {
        for (int d = tid; d < D; d += 256) orow[d] = __builtin_nanf("");
        return;
    }
    // exponentials: the vector part through Cephes, the tail through f64 exp
    const int64_t nv = n >= 8 ? (n & ~(int64_t)7) : 0;
    for (int64_t j = tid; j < n; j += 256) {
        const float x = sc[j] - mx;
        sc[j] = j < nv ? cephes_exp(x) : (float)exp((double)x);
    }
    __syncthreads();
    if (tid < 8) {
        float s = 0.f;
        for (int64_t j = tid; j < nv; j += 8) s = s + sc[j];
        lane_sum[tid] = s;
    }
    __syncthreads();
    float sum = ((lane_sum[0] + lane_sum[4]) + (lane_sum[1] + lane_sum[5])) +
                ((lane_sum[2] + lane_sum[6]) + (lane_sum[3] + lane_sum[7]));
    if (nv == 0) sum = 0.f;
    for (int64_t j = nv; j < n; j++) sum = sum + sc[j];
    // o[d] = (sum_j e_j v_j[d]) / sum, the keys in order
    for (int d = tid; d < D; d += 256) {
        const int64_t vb = cbase * D + d;
        float acc = 0.f;
        int64_t j = 0;
        for (; j + 4 <= n; j += 4) {
            const float v0 = kv_at(vc, vb + (j + 0) * D, f16), v1 = kv_at(vc, vb + (j + 1) * D, f16);
            const float v2 = kv_at(vc, vb + (j + 2) * D, f16), v3 = kv_at(vc, vb + (j + 3) * D, f16);
            acc = __builtin_fmaf(sc[j], v0, acc);
            acc = __builtin_fmaf(sc[j + 1], v1, acc);
            acc = __builtin_fmaf(sc[j + 2], v2, acc);
            acc = __builtin_fmaf(sc[j + 3], v3, acc);
        }
        for (; j < n; j++) acc = __builtin_fmaf(sc[j], kv_at(vc, vb + j * D, f16), acc);
        orow[d] = acc / sum;
    }
}

// silu(x) * b as the reference's siluMulF32AVX2 (attn_amd64.s:459-535):
// h = exp(-|x|/2) by the Cephes steps, silu = x/(1+h*h) for x >= 0 and
// ((x*h)*h)/(1+h*h) below, then times b.
__device__ __forceinline__ float silu_mul_vec(float x, float b) {
    const float hh = cephes_exp(-__builtin_fabsf(x) * 0.5f);
    const float e1 = hh * hh + 1.0f;
    const float y = (x * hh) * hh;
    return ((x >= 0.f ? x : y) / e1) * b;
}

// swiglu.v1 (reference interp/fast.go:487-498): the reference splits the n
// elements into pieces of `chunk` (parallel(), interp/pool.go:33-51, 79-97)
// and runs SiluMulF32 (attn.go:63-76) on each: the first len&~7 elements of
// a piece through the vector formula, the rest as
// f32(f64(g)/(1+exp(-f64(g)))*f64(u)).
__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out, int64_t n,
                              int64_t chunk) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t lo = i / chunk * chunk;
        const int64_t len = lo + chunk < n ? chunk : n - lo;
        const int64_t nv = len >= 8 ? (len & ~(int64_t)7) : 0;
        const float x = g[i], y = u[i];
        if (i - lo < nv) {
            out[i] = silu_mul_vec(x, y);
        } else {
            const double a = (double)x;
            out[i] = (float)(a / (1.0 + exp(-a)) * (double)y);
        }
    }
}

// One 1024-thread workgroup per row of logits: the first index of the max.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t n, int32_t* __restrict__ out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float* r = x + (int64_t)blockIdx.x * n;
    float best = -INFINITY;
    int idx = (int)n;  // none yet
    for (int i = threadIdx.x; i < (int)n; i += 1024) {
        const float v = r[i];
        if (idx == n || v > best) {
            best = v;
            idx = i;
        }
    }
    // lexicographic (larger value, then smaller index) across the group
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(idx, off);
        if (oi < n && (idx == n || ov > best || (ov == best && oi < idx))) {
            best = ov;
            idx = oi;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[w] = best;
        bi[w] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int i0 = bi[0];
        for (int k = 1; k < 16; k++)
            if (bi[k] < n && (i0 == n || bv[k] > b || (bv[k] == b && bi[k] < i0))) {
                b = bv[k];
                i0 = bi[k];
            }
        out[blockIdx.x] = (int32_t)(i0 == n ? 0 : i0);
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

hipError_t launch_attention(const float* q, const void* kc, const void* vc, const int64_t* kend, const int64_t* kstart,
                            int T, int H, int Hkv, int D, int64_t C, int f16, float* out, hipStream_t s) {
    if (D > 512 || D % 8 || H % Hkv) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)H, (unsigned)T), dim3(256), 0, s, q, kc, vc, kend, kstart, H, Hkv,
                       D, C, f16, out);
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
