// The ops around the linear layers in a llama/qwen2 decoder step, on the
// GPU so that a step's activations stay in device memory: the other fast
// paths of the graph BuildLlama writes (reference importer/llama.go:317-547,
// interp/fast.go:40-59). Their float results follow the reference's
// formulas; the checks are the reference fixture's tolerances against its
// float64 oracle (not bits: the reference computes several of them with
// vector kernels whose lane order and exp polynomials are not pinned).
//
//   embedding.v1  rows of the table decoded exactly (interp/fast.go:818-842)
//   rms_norm.v1   f64 sum of squares; inv = f32(1/sqrt(f64(f32(ss/n)) +
//                 f64(f32(eps)))); y = (x*inv)*scale (interp/fast.go:434-485)
//   rope.v1       angles pos*invFreq_i in f64, c = f32(cos), s = f32(sin),
//                 x1*c - x2*s, x2*c + x1*s in f32 (interp/fast.go:507-557)
//   attention.v1/2  keys j <= position visible; scores f32(q.k)*f32(1/sqrt(D));
//                 e = f32(exp(f64(s - max))); o = (sum e*v) / sum e
//                 (interp/fast.go:569-700); with the cache in f16, keys and
//                 values are rounded to f16 as they are stored
//   swiglu.v1     f32(f64(g)/(1+exp(-f64(g)))*f64(u)) (internal/kernels/attn.go:63-73)
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

// One 256-thread workgroup per (query t, head h): cache entries
// kstart[t]..kend[t] (inclusive; kstart 0 when null) of kv head h / (H / Hkv).
// Scores go through LDS (at most ATT_MAXC visible keys).
constexpr int ATT_MAXC = 8192;
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q, const void* kc, const void* vc,
                                                        const int64_t* __restrict__ kend,
                                                        const int64_t* __restrict__ kstart, int H, int Hkv, int D,
                                                        int64_t C, int f16, float* __restrict__ out) {
    __shared__ float sc[ATT_MAXC];
    __shared__ float qs[512];
    __shared__ float red[4];
    __shared__ float accs[4][512];
    const int t = blockIdx.y, h = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int hk = h / (H / Hkv);
    // visible keys, indexed from k0; kept inside the cache row and LDS
    const int64_t k0 = kstart ? (kstart[t] < 0 ? 0 : (kstart[t] >= C ? C - 1 : kstart[t])) : 0;
    int64_t end = kend[t] + 1 - k0;
    if (end > C - k0) end = C - k0;
    if (end > ATT_MAXC) end = ATT_MAXC;
    const int64_t cbase = (int64_t)hk * C + k0;
    const float scale = (float)(1.0 / sqrt((double)D));
    const float* qr = q + ((int64_t)t * H + h) * D;
    for (int d = tid; d < D; d += 256) qs[d] = qr[d];
    __syncthreads();
    // scores: a wave per key, lanes over D
    for (int64_t j = w; j < end; j += 4) {
        const int64_t base = (cbase + j) * D;
        float part = 0.f;
        for (int d = lane; d < D; d += 64) part = __builtin_fmaf(qs[d], kv_at(kc, base + d, f16), part);
        part = wave_sum_f32(part);
        if (lane == 0) sc[j] = part * scale;
    }
    __syncthreads();
    float* orow = out + ((int64_t)t * H + h) * D;
    if (end <= 0) {  // nothing visible
        for (int d = tid; d < D; d += 256) orow[d] = 0.f;
        return;
    }
    float mx = -INFINITY;
    for (int64_t j = tid; j < end; j += 256) mx = fmaxf(mx, sc[j]);
    mx = wave_max_f32(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int64_t j = tid; j < end; j += 256) {
        const float e = (float)exp((double)(sc[j] - mx));
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum_f32(sum);
    if (lane == 0) red[w] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);
    // o[d] = sum_j e_j v_j[d] / sum: the waves split the keys, lanes the dims
    for (int d0 = 0; d0 < D; d0 += 64) {
        const int d = d0 + lane;
        float acc = 0.f;
        if (d < D)
            for (int64_t j = w; j < end; j += 4) acc = __builtin_fmaf(sc[j], kv_at(vc, (cbase + j) * D + d, f16), acc);
        if (d < D) accs[w][d] = acc;
    }
    __syncthreads();
    for (int d = tid; d < D; d += 256) orow[d] = ((accs[0][d] + accs[1][d]) + (accs[2][d] + accs[3][d])) / sum;
}

__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const double a = (double)g[i];
        out[i] = (float)(a / (1.0 + exp(-a)) * (double)u[i]);
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
    if (D > 512 || H % Hkv) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)H, (unsigned)T), dim3(256), 0, s, q, kc, vc, kend, kstart, H, Hkv,
                       D, C, f16, out);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* out, int64_t n, hipStream_t s) {
    const unsigned grid = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid ? grid : 1), dim3(256), 0, s, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int64_t rows, int64_t n, int32_t* out, hipStream_t s) {
    if (n <= 0 || n >= (1ll << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, s, x, n, out);
    return hipGetLastError();
}

}  // namespace mimg
