// Block encoders on the GPU, for synthetic weights (f32 -> block bytes).
//
// Q8_0 is the reference encoder (quant.go:208-228, ggml
// quantize_row_q8_0_ref): d = amax/127, id = 1/d, q = round-half-away(x*id).
// The reference has no Q4_K/Q6_K encoder (quant.go:165-194); encoders are
// not normative (spec/dtypes.md:44-45), so these are this repository's own:
//   Q4_K: per 32-element sub-block scale (max-min)/15 and offset -min (min
//         clamped to <= 0); d = max scale/63, dmin = max offset/63 as f16;
//         6-bit scales/offsets and 4-bit quants rounded to nearest even
//         against the decoded f16 values.
//   Q6_K: per 16-element sub-block scale max|x|/31; d = max scale/127 as f16;
//         int8 scales and quants in -32..31, rounded to nearest even.
// One thread per block. The same float operations as the CPU oracle's
// encoders, so both give identical bytes (checked by the tests).
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

namespace mimg {

// float -> f16 bits, round to nearest even (reference F32ToF16, float.go:46-84).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

__global__ void encode_q8_0_kernel(const float* __restrict__ x, int64_t nb, uint8_t* __restrict__ dst) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* xb = x + 32 * b;
    float amax = 0.f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
    float d = amax / 127.0f;
    float id = d != 0.f ? 1.0f / d : 0.0f;
    uint8_t* blk = dst + 34 * b;
    uint16_t h = f32_to_f16(d);
    blk[0] = (uint8_t)h;
    blk[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) blk[2 + j] = (uint8_t)(int8_t)(int)roundf(xb[j] * id);
}

__global__ void encode_q4_k_kernel(const float* __restrict__ src, int64_t nb, uint8_t* __restrict__ dst) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* x = src + 256 * b;
    uint8_t* blk = dst + 144 * b;
    float scale[8], offs[8], maxs = 0.f, maxo = 0.f;
    for (int s = 0; s < 8; s++) {
        float mn = x[32 * s], mx = x[32 * s];
        for (int i = 1; i < 32; i++) {
            float v = x[32 * s + i];
            mn = v < mn ? v : mn;
            mx = v > mx ? v : mx;
        }
        if (mn > 0.f) mn = 0.f;
        scale[s] = (mx - mn) / 15.0f;
        offs[s] = -mn;
        maxs = scale[s] > maxs ? scale[s] : maxs;
        maxo = offs[s] > maxo ? offs[s] : maxo;
    }
    uint16_t hd = f32_to_f16(maxs / 63.0f), hm = f32_to_f16(maxo / 63.0f);
    float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    int sc[8], m[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = d > 0.f ? clampi((int)__builtin_rintf(scale[s] / d), 0, 63) : 0;
        m[s] = dmin > 0.f ? clampi((int)__builtin_rintf(offs[s] / dmin), 0, 63) : 0;
    }
    blk[0] = (uint8_t)hd;
    blk[1] = (uint8_t)(hd >> 8);
    blk[2] = (uint8_t)hm;
    blk[3] = (uint8_t)(hm >> 8);
    for (int j = 0; j < 4; j++) {
        blk[4 + j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        blk[8 + j] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        blk[12 + j] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    for (int c = 0; c < 4; c++) {
        float ds0 = d * (float)sc[2 * c], ms0 = dmin * (float)m[2 * c];
        float ds1 = d * (float)sc[2 * c + 1], ms1 = dmin * (float)m[2 * c + 1];
        for (int l = 0; l < 32; l++) {
            int q0 = ds0 > 0.f ? clampi((int)__builtin_rintf((x[64 * c + l] + ms0) / ds0), 0, 15) : 0;
            int q1 = ds1 > 0.f ? clampi((int)__builtin_rintf((x[64 * c + 32 + l] + ms1) / ds1), 0, 15) : 0;
            blk[16 + 32 * c + l] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

__global__ void encode_q6_k_kernel(const float* __restrict__ src, int64_t nb, uint8_t* __restrict__ dst) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* x = src + 256 * b;
    uint8_t* blk = dst + 210 * b;
    float scale[16], maxs = 0.f;
    for (int s = 0; s < 16; s++) {
        float a = 0.f;
        for (int i = 0; i < 16; i++) {
            float v = fabsf(x[16 * s + i]);
            a = v > a ? v : a;
        }
        scale[s] = a / 31.0f;
        maxs = scale[s] > maxs ? scale[s] : maxs;
    }
    uint16_t hd = f32_to_f16(maxs / 127.0f);
    float d = f16_to_f32(hd);
    int sc[16];
    for (int s = 0; s < 16; s++) sc[s] = d > 0.f ? clampi((int)__builtin_rintf(scale[s] / d), -128, 127) : 0;
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            int q[4];
            for (int p = 0; p < 4; p++) {
                int e = 128 * h + 32 * p + l;
                float ds = d * (float)sc[e / 16];
                q[p] = (ds != 0.f ? clampi((int)__builtin_rintf(x[e] / ds), -32, 31) : 0) + 32;
            }
            blk[64 * h + l] = (uint8_t)((q[0] & 15) | ((q[2] & 15) << 4));
            blk[64 * h + 32 + l] = (uint8_t)((q[1] & 15) | ((q[3] & 15) << 4));
            blk[128 + 32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
        }
    for (int s = 0; s < 16; s++) blk[192 + s] = (uint8_t)(int8_t)sc[s];
    blk[208] = (uint8_t)hd;
    blk[209] = (uint8_t)(hd >> 8);
}

// Synthetic N(0, std^2) values for benchmark models: element pair i comes
// from one 64-bit hash of (seed, i) (splitmix64's finaliser) through the
// Box-Muller transform, so the values depend on (seed, i) only, not on the
// launch shape.
__device__ __forceinline__ uint64_t splitmix_fin(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void normal_fill_kernel(uint64_t seed, float stdv, float* __restrict__ dst, int64_t n) {
    const int64_t pairs = (n + 1) / 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs; i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t h = splitmix_fin(splitmix_fin(seed) ^ (0x9e3779b97f4a7c15ull * (uint64_t)(i + 1)));
        const float u1 = (float)((h >> 40) + 1) * 0x1p-24f;     // (0, 1]
        const float u2 = (float)((h >> 16) & 0xFFFFFF) * 0x1p-24f;  // [0, 1)
        const float r = stdv * sqrtf(-2.f * logf(u1));
        float sn, cs;
        sincosf(6.2831853f * u2, &sn, &cs);
        dst[2 * i] = r * cs;
        if (2 * i + 1 < n) dst[2 * i + 1] = r * sn;
    }
}

hipError_t launch_normal_fill(uint64_t seed, float stdv, float* dst, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t pairs = (n + 1) / 2;
    const unsigned grid = (unsigned)((pairs + 255) / 256 < 16384 ? (pairs + 255) / 256 : 16384);
    hipLaunchKernelGGL(normal_fill_kernel, dim3(grid), dim3(256), 0, stream, seed, stdv, dst, n);
    return hipGetLastError();
}

hipError_t launch_encode(uint32_t dt, const float* x, int64_t n, uint8_t* dst, hipStream_t stream) {
    int64_t be = dt == DT_Q8_0 ? 32 : 256;
    int64_t nb = n / be;
    if (nb <= 0) return hipSuccess;
    dim3 grid((unsigned)((nb + 127) / 128)), blk(128);
    switch (dt) {
    case DT_Q8_0: hipLaunchKernelGGL(encode_q8_0_kernel, grid, blk, 0, stream, x, nb, dst); break;
    case DT_Q4_K: hipLaunchKernelGGL(encode_q4_k_kernel, grid, blk, 0, stream, x, nb, dst); break;
    case DT_Q6_K: hipLaunchKernelGGL(encode_q6_k_kernel, grid, blk, 0, stream, x, nb, dst); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mimg
