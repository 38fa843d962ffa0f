/*
 * mimref.c — CPU restatement of the reference numerics (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libmimg.so, loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
 * product path.
 *
 * Written from the reference's text (file:line cited per function), not
 * translated: the float32 operation order is the contract, so each function
 * states the order it follows. Built with -ffp-contract=off so that every
 * multiply and add rounds on its own unless fmaf() is written.
 *
 * Parity pins (tests/test_oracle.py):
 *   f16 decode, Q8_0/Q4_K/Q6_K decode ... testdata/quant_golden.json bits,
 *        conformance dequantize.json, hand-built known answers, exhaustive
 *        f16 check against numpy's float16.
 *   Q8_0 encoder ....................... quant_golden.json input_bits/bytes.
 *   activation quantizer ............... known answers (q8_test.go:58-85),
 *        brute force against exact rational rounding.
 *   block-256 a8 dots .................. the closed form of dotQ8KRef
 *        (q8k_test.go:38-102) evaluated independently in Python with exact
 *        integers and exactly-rounded float32 FMA, plus its special inputs.
 *   block-32 a8 dots, f32 dots ......... lane order restated from
 *        kernels_amd64.s; pinned only up to the spec tolerance and a float64
 *        brute force (parity unpinned at the bit level: no golden output of
 *        the AVX2 kernels exists and Go cannot run here).
 *   Q4_K/Q6_K encoders ................. non-normative (spec/dtypes.md:44-45);
 *        checked by round trip (decode within one step of the input).
 */
#include "mimref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float mref_fmaf(float a, float b, float c) { return fmaf(a, b, c); }

/* F16ToF32, float.go:24-44: exact, subnormals normalised. */
float mref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign);
        uint32_t e = 127 - 15 + 1;
        while ((mant & 0x400u) == 0) {
            mant <<= 1;
            e--;
        }
        return bits_f32(sign | e << 23 | (mant & 0x3FFu) << 13);
    }
    if (exp == 0x1F) return bits_f32(sign | 0x7F800000u | mant << 13);
    return bits_f32(sign | (exp + 127 - 15) << 23 | mant << 13);
}

void mref_f16_to_f32_n(const uint16_t *h, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = mref_f16_to_f32(h[i]);
}

/* F32ToF16, float.go:46-84: round to nearest even. */
uint16_t mref_f32_to_f16(float f) {
    uint32_t b = f32_bits(f);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xFF);
    uint32_t mant = b & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (mant == 0) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | (mant >> 13));
    }
    int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -11) return sign;
        mant |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = mant & ((half << 1) - 1);
        uint32_t q = mant >> shift;
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (uint32_t)e << 10 | mant >> 13;
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++; /* may carry to inf: correct */
    return (uint16_t)(sign | q);
}

int64_t mref_block_elems(uint32_t dt) {
    switch (dt) {
    case MREF_F32: return 1;
    case MREF_Q8_0: return 32;
    case MREF_Q4_K:
    case MREF_Q6_K: return 256;
    }
    return -1;
}

int64_t mref_block_bytes(uint32_t dt) {
    switch (dt) {
    case MREF_F32: return 4;
    case MREF_Q8_0: return 34;
    case MREF_Q4_K: return 144;
    case MREF_Q6_K: return 210;
    }
    return -1;
}

int64_t mref_row_bytes(uint32_t dt, int64_t k) {
    int64_t be = mref_block_elems(dt);
    if (be <= 0 || k < 0 || k % be) return -1;
    return k / be * mref_block_bytes(dt);
}

/* ---------------------------------------------------------------- decode */

/* dequantizeQ8_0, quant.go:197-206: y = d*q. */
static void deq_q8_0(const uint8_t *src, float *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + 34 * b;
        float d = mref_f16_to_f32(le16(blk));
        for (int j = 0; j < 32; j++) dst[32 * b + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* getScaleMinK4, quant.go:272-281 (spec/dtypes.md:187-196). */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequantizeQ4_K, quant.go:283-313: y = f32(d*sc)*q - f32(dmin*m), two roundings each. */
static void deq_q4_k(const uint8_t *src, float *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + 144 * b;
        float d = mref_f16_to_f32(le16(blk));
        float dmin = mref_f16_to_f32(le16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *q = blk + 16;
        float *y = dst + 256 * b;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            scale_min_k4(2 * c, scales, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, scales, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; l++) y[64 * c + l] = d1 * (float)(q[32 * c + l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
        }
    }
}

/* Q6_K quant l of half h (spec/dtypes.md:228-246), minus 32. */
static inline int q6_quant(const uint8_t *blk, int h, int part, int l) {
    const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
    int v;
    switch (part) {
    case 0: v = (ql[l] & 0xF) | ((qh[l] & 3) << 4); break;
    case 1: v = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4); break;
    case 2: v = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4); break;
    default: v = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4); break;
    }
    return v - 32;
}

/* dequantizeQ6_K, quant.go:315-344: y = f32(d*sc)*(q-32). */
static void deq_q6_k(const uint8_t *src, float *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + 210 * b;
        float d = mref_f16_to_f32(le16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        float *y = dst + 256 * b;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                for (int p = 0; p < 4; p++) {
                    float s = d * (float)sc[8 * h + is + 2 * p];
                    y[128 * h + 32 * p + l] = s * (float)q6_quant(blk, h, p, l);
                }
            }
    }
}

/* Dequantize, quant.go:37-73: size checks, then block decode. */
int mref_dequantize(uint32_t dt, const uint8_t *src, int64_t src_len, float *dst, int64_t n) {
    int64_t be = mref_block_elems(dt);
    if (be < 0) return MREF_ERR_DTYPE;
    if (n < 0 || n % be) return MREF_ERR_SIZE;
    if (n / be * mref_block_bytes(dt) != src_len) return MREF_ERR_SIZE;
    switch (dt) {
    case MREF_F32: memcpy(dst, src, (size_t)n * 4); break;
    case MREF_Q8_0: deq_q8_0(src, dst, n / 32); break;
    case MREF_Q4_K: deq_q4_k(src, dst, n / 256); break;
    case MREF_Q6_K: deq_q6_k(src, dst, n / 256); break;
    default: return MREF_ERR_DTYPE;
    }
    return MREF_OK;
}

/* ---------------------------------------------------------------- encode */

/* quantizeQ8_0, quant.go:208-228 (ggml quantize_row_q8_0_ref): d = amax/127,
 * id = 1/d, q = round-half-away(x*id). Pinned by quant_golden.json. */
static void enc_q8_0(const float *src, uint8_t *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float *x = src + 32 * b;
        float amax = 0;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0 ? 1.0f / d : 0.0f;
        uint8_t *blk = dst + 34 * b;
        uint16_t h = mref_f32_to_f16(d);
        blk[0] = (uint8_t)h;
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            float v = x[j] * id;
            blk[2 + j] = (uint8_t)(int8_t)(float)round((double)v);
        }
    }
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* Q4_K encoder — this repository's own, non-normative (spec/dtypes.md:44-45;
 * the reference has none, quant.go:165-194). Per 32-element sub-block an
 * asymmetric min/max fit: scale (max-min)/15 and offset -min (min clamped to
 * <= 0); the 6-bit scales and offsets are those over the super-block maxima
 * d = max scale/63, dmin = max offset/63 (stored as f16); the quants are then
 * rounded against the decoded f16 values and clamped to 0..15. */
static void enc_q4_k(const float *src, uint8_t *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float *x = src + 256 * b;
        uint8_t *blk = dst + 144 * b;
        float scale[8], offs[8];
        float maxs = 0, maxo = 0;
        for (int s = 0; s < 8; s++) {
            float mn = x[32 * s], mx = x[32 * s];
            for (int i = 1; i < 32; i++) {
                float v = x[32 * s + i];
                if (v < mn) mn = v;
                if (v > mx) mx = v;
            }
            if (mn > 0) mn = 0;
            scale[s] = (mx - mn) / 15.0f;
            offs[s] = -mn;
            if (scale[s] > maxs) maxs = scale[s];
            if (offs[s] > maxo) maxo = offs[s];
        }
        uint16_t hd = mref_f32_to_f16(maxs / 63.0f), hm = mref_f32_to_f16(maxo / 63.0f);
        float d = mref_f16_to_f32(hd), dmin = mref_f16_to_f32(hm);
        int sc[8], m[8];
        for (int s = 0; s < 8; s++) {
            sc[s] = d > 0 ? clampi((int)lrintf(scale[s] / d), 0, 63) : 0;
            m[s] = dmin > 0 ? clampi((int)lrintf(offs[s] / dmin), 0, 63) : 0;
        }
        memset(blk, 0, 144);
        blk[0] = (uint8_t)hd;
        blk[1] = (uint8_t)(hd >> 8);
        blk[2] = (uint8_t)hm;
        blk[3] = (uint8_t)(hm >> 8);
        uint8_t *s12 = blk + 4;
        for (int j = 0; j < 4; j++) {
            s12[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int s = 0; s < 8; s++) {
            float ds = d * (float)sc[s], ms = dmin * (float)m[s];
            for (int i = 0; i < 32; i++) {
                int v = ds > 0 ? clampi((int)lrintf((x[32 * s + i] + ms) / ds), 0, 15) : 0;
                q[32 * s + i] = (uint8_t)v;
            }
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++)
                blk[16 + 32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
    }
}

/* Q6_K encoder — this repository's own, non-normative. Per 16-element
 * sub-block a symmetric fit, scale max|x|/31; the int8 scales over
 * d = max scale/127 (f16); quants rounded against the decoded scales and
 * clamped to -32..31, stored +32 in the ql/qh layout of spec/dtypes.md:228-246. */
static void enc_q6_k(const float *src, uint8_t *dst, int64_t nb) {
    for (int64_t b = 0; b < nb; b++) {
        const float *x = src + 256 * b;
        uint8_t *blk = dst + 210 * b;
        float scale[16], maxs = 0;
        for (int s = 0; s < 16; s++) {
            float a = 0;
            for (int i = 0; i < 16; i++) {
                float v = fabsf(x[16 * s + i]);
                if (v > a) a = v;
            }
            scale[s] = a / 31.0f;
            if (scale[s] > maxs) maxs = scale[s];
        }
        uint16_t hd = mref_f32_to_f16(maxs / 127.0f);
        float d = mref_f16_to_f32(hd);
        int sc[16];
        for (int s = 0; s < 16; s++) sc[s] = d > 0 ? clampi((int)lrintf(scale[s] / d), -128, 127) : 0;
        memset(blk, 0, 210);
        int q[256];
        for (int e = 0; e < 256; e++) {
            float ds = d * (float)sc[e / 16];
            q[e] = ds != 0 ? clampi((int)lrintf(x[e] / ds), -32, 31) : 0;
        }
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                int q1 = q[128 * h + l] + 32, q2 = q[128 * h + 32 + l] + 32;
                int q3 = q[128 * h + 64 + l] + 32, q4 = q[128 * h + 96 + l] + 32;
                blk[64 * h + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                blk[64 * h + 32 + l] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                blk[128 + 32 * h + l] =
                    (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int s = 0; s < 16; s++) blk[192 + s] = (uint8_t)(int8_t)sc[s];
        blk[208] = (uint8_t)hd;
        blk[209] = (uint8_t)(hd >> 8);
    }
}

int mref_quantize(uint32_t dt, const float *src, int64_t n, uint8_t *dst, int64_t dst_len) {
    int64_t be = mref_block_elems(dt);
    if (be < 0 || dt == MREF_F32) return MREF_ERR_DTYPE;
    if (n < 0 || n % be) return MREF_ERR_SIZE;
    if (n / be * mref_block_bytes(dt) != dst_len) return MREF_ERR_SIZE;
    switch (dt) {
    case MREF_Q8_0: enc_q8_0(src, dst, n / 32); break;
    case MREF_Q4_K: enc_q4_k(src, dst, n / 256); break;
    case MREF_Q6_K: enc_q6_k(src, dst, n / 256); break;
    default: return MREF_ERR_DTYPE;
    }
    return MREF_OK;
}

/* ------------------------------------------------- activation quantizer */

/* Q8.QuantizeBlocks, q8.go:50-97 with amaxQ8Go/quantQ8Go/sumsQ8Go
 * (q8.go:237-273): per block amax = max|x|, refused if any |x| is NaN or
 * above 2^60; q = RoundToEven(127*f64(x)/f64(amax)) (0 when amax == 0);
 * d = f32(amax)/127 repeated for each run of 32; xs = sum of each run of 32;
 * m32[i] = 32*(q[2i]+q[2i+1]); dbs = d*f32(xs). */
int mref_quantize_act(const float *x, int64_t k, int block, int8_t *q, float *d, int16_t *xs,
                      int16_t *m32, float *dbs) {
    if (k <= 0 || (block != 32 && block != 256) || k % block) return 0;
    for (int64_t b = 0; b < k / block; b++) {
        const float *xb = x + block * b;
        float amax = 0;
        for (int i = 0; i < block; i++) {
            float a = bits_f32(f32_bits(xb[i]) & 0x7FFFFFFFu);
            if (!(a <= 0x1p60f)) return 0;
            if (a > amax) amax = a;
        }
        int8_t *qb = q + block * b;
        for (int i = 0; i < block; i++)
            qb[i] = amax == 0 ? 0 : (int8_t)nearbyint(127.0 * (double)xb[i] / (double)amax);
        float dd = amax / 127.0f;
        for (int64_t r = block * b / 32; r < block * (b + 1) / 32; r++) {
            int s = 0;
            for (int i = 0; i < 32; i++) s += q[32 * r + i];
            if (xs) xs[r] = (int16_t)s;
            if (d) d[r] = dd;
            if (dbs) dbs[r] = dd * (float)(int16_t)s;
        }
        if (m32)
            for (int64_t i = block * b / 2; i < block * (b + 1) / 2; i++)
                m32[i] = (int16_t)(32 * (q[2 * i] + q[2 * i + 1]));
    }
    return 1;
}

/* ---------------------------------------------------- 8-bit dot products */

static inline int f16_finite(const uint8_t *p) { return (le16(p) & 0x7C00u) != 0x7C00u; }

/* dotQ8KRef for Q4_K, q8k_test.go:38-76 (= dotQ4KQ8KAVX2, kernels_amd64.s:1141-1224):
 * per block exact int32 S = sum_s sc_s * sum q*y and M = sum_j m_j*xs_j, then
 * tot = fma(f32(S), d*dx, tot), off = fma(f32(M), dmin*dx, off) in block order;
 * the result is tot - off. dx is the block's d, read at its first run of 32. */
int mref_dot_q4k_a8k(const uint8_t *row, const int8_t *y0, const float *dxs, const int16_t *xs,
                     int64_t nb, float *out) {
    float tot = 0, off = 0;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 144 * b;
        if (!f16_finite(blk) || !f16_finite(blk + 2)) return 0;
        float d = mref_f16_to_f32(le16(blk)), dmin = mref_f16_to_f32(le16(blk + 2));
        float dx = dxs[8 * b];
        const int8_t *y = y0 + 256 * b;
        int32_t S = 0, M = 0;
        for (int c = 0; c < 4; c++) {
            uint8_t sc0, m0, sc1, m1;
            scale_min_k4(2 * c, blk + 4, &sc0, &m0);
            scale_min_k4(2 * c + 1, blk + 4, &sc1, &m1);
            int32_t lo = 0, hi = 0;
            for (int i = 0; i < 32; i++) {
                uint8_t v = blk[16 + 32 * c + i];
                lo += (int32_t)(v & 15) * y[64 * c + i];
                hi += (int32_t)(v >> 4) * y[64 * c + 32 + i];
            }
            S += (int32_t)sc0 * lo + (int32_t)sc1 * hi;
        }
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            scale_min_k4(j, blk + 4, &sc, &m);
            M += (int32_t)m * xs[8 * b + j];
        }
        tot = fmaf((float)S, d * dx, tot);
        off = fmaf((float)M, dmin * dx, off);
    }
    *out = tot - off;
    return 1;
}

/* dotQ8KRef for Q6_K, q8k_test.go:78-101 (= dotQ6KQ8KAVX2, kernels_amd64.s:1369-1435):
 * exact S = sum sc_i8*(q-32)*y per block, tot = fma(f32(S), d*dx, tot). */
int mref_dot_q6k_a8k(const uint8_t *row, const int8_t *y0, const float *dxs, int64_t nb,
                     float *out) {
    float tot = 0;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 210 * b;
        if (!f16_finite(blk + 208)) return 0;
        float d = mref_f16_to_f32(le16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const int8_t *y = y0 + 256 * b;
        int32_t S = 0;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                for (int p = 0; p < 4; p++)
                    S += (int32_t)sc[8 * h + is + 2 * p] * q6_quant(blk, h, p, l) * y[128 * h + 32 * p + l];
            }
        tot = fmaf((float)S, d * dxs[8 * b], tot);
    }
    *out = tot;
    return 1;
}

/* HSUM1 of kernels_amd64.s:405-411 over eight lanes: ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)). */
static inline float hsum8(const float a[8]) {
    float c0 = a[0] + a[4], c1 = a[1] + a[5], c2 = a[2] + a[6], c3 = a[3] + a[7];
    return (c0 + c1) + (c2 + c3);
}

/* dotQ8_0Q8AVX2, kernels_amd64.s:1003-1043: lane l of block b holds the exact
 * sum P of elements 4l..4l+3, acc_l = fma(f32(P), f32(d_w*dx_b), acc_l) in
 * block order, then HSUM1. Lane order from the asm text (bit parity unpinned). */
int mref_dot_q8_0_a8(const uint8_t *row, const int8_t *y, const float *dx, int64_t nb, float *out) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 34 * b;
        if (!f16_finite(blk)) return 0;
        float s = mref_f16_to_f32(le16(blk)) * dx[b];
        for (int l = 0; l < 8; l++) {
            int32_t P = 0;
            for (int t = 0; t < 4; t++) P += (int32_t)(int8_t)blk[2 + 4 * l + t] * y[32 * b + 4 * l + t];
            acc[l] = fmaf((float)P, s, acc[l]);
        }
    }
    *out = hsum8(acc);
    return 1;
}

/* dotQ4KQ8AVX2 (activation blocks of 32), kernels_amd64.s:428-597. Per block:
 * lanes i of the chunk sums A (sub-block 2c) and B (2c+1) get
 * fma(f32(sc*sum_{4i..4i+3} q*y), dx_run, .) over c = 0..3; then
 * tot_i = fma(d, A_i+B_i, tot_i) and off_j = fma(dmin*m_j, dbs_j, off_j);
 * the result is HSUM1(tot - off). Bit parity unpinned (lane order from asm). */
int mref_dot_q4k_a8(const uint8_t *row, const int8_t *y0, const float *dx, const float *dbs,
                    int64_t nb, float *out) {
    float tot[8] = {0}, off[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 144 * b;
        if (!f16_finite(blk) || !f16_finite(blk + 2)) return 0;
        float d = mref_f16_to_f32(le16(blk)), dmin = mref_f16_to_f32(le16(blk + 2));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            scale_min_k4(j, blk + 4, &sc, &m);
            off[j] = fmaf(dmin * (float)m, dbs[8 * b + j], off[j]);
        }
        float A[8] = {0}, B[8] = {0};
        const int8_t *y = y0 + 256 * b;
        for (int c = 0; c < 4; c++) {
            uint8_t sc0, m0, sc1, m1;
            scale_min_k4(2 * c, blk + 4, &sc0, &m0);
            scale_min_k4(2 * c + 1, blk + 4, &sc1, &m1);
            for (int i = 0; i < 8; i++) {
                int32_t lo = 0, hi = 0;
                for (int t = 0; t < 4; t++) {
                    uint8_t v = blk[16 + 32 * c + 4 * i + t];
                    lo += (int32_t)(v & 15) * y[64 * c + 4 * i + t];
                    hi += (int32_t)(v >> 4) * y[64 * c + 32 + 4 * i + t];
                }
                A[i] = fmaf((float)(sc0 * lo), dx[8 * b + 2 * c], A[i]);
                B[i] = fmaf((float)(sc1 * hi), dx[8 * b + 2 * c + 1], B[i]);
            }
        }
        for (int i = 0; i < 8; i++) tot[i] = fmaf(d, A[i] + B[i], tot[i]);
    }
    float r[8];
    for (int i = 0; i < 8; i++) r[i] = tot[i] - off[i];
    *out = hsum8(r);
    return 1;
}

/* dotQ6KQ8AVX2 (activation blocks of 32), kernels_amd64.s:760-882. Per half h
 * and quarter p, lane i holds sc*(sum over elements 4i..4i+3 of the quarter of
 * (q-32)*y) (scale sc[8h+2p+i/4]); quarters 0,2 go to A and 1,3 to B with
 * fma(f32(.), dx_run, .); then tot_i = fma(d, A_i+B_i, tot_i); HSUM1(tot).
 * Bit parity unpinned (lane order from asm). */
int mref_dot_q6k_a8(const uint8_t *row, const int8_t *y0, const float *dx, const int16_t *m32,
                    int64_t nb, float *out) {
    (void)m32; /* the asm subtracts 32*(y pair) via m32; the integer result is the same */
    float tot[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 210 * b;
        if (!f16_finite(blk + 208)) return 0;
        float d = mref_f16_to_f32(le16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const int8_t *y = y0 + 256 * b;
        float A[8] = {0}, B[8] = {0};
        for (int h = 0; h < 2; h++)
            for (int p = 0; p < 4; p++)
                for (int i = 0; i < 8; i++) {
                    int32_t s = 0;
                    for (int t = 0; t < 4; t++) {
                        int l = 4 * i + t;
                        s += q6_quant(blk, h, p, l) * y[128 * h + 32 * p + l];
                    }
                    int32_t v = (int32_t)sc[8 * h + 2 * p + i / 4] * s;
                    float dd = dx[8 * b + 4 * h + p];
                    if (p % 2 == 0) A[i] = fmaf((float)v, dd, A[i]);
                    else B[i] = fmaf((float)v, dd, B[i]);
                }
        for (int i = 0; i < 8; i++) tot[i] = fmaf(d, A[i] + B[i], tot[i]);
    }
    *out = hsum8(tot);
    return 1;
}

/* --------------------------------------------- float32 dot products */

/* HSUM of kernels_amd64.s:28-37 over four 8-lane accumulators:
 * T = (Y0+Y1)+(Y2+Y3) lane-wise, then ((T0+T4)+(T1+T5))+((T2+T6)+(T3+T7)). */
static inline float hsum32(float Y[4][8]) {
    float T[8];
    for (int l = 0; l < 8; l++) T[l] = (Y[0][l] + Y[1][l]) + (Y[2][l] + Y[3][l]);
    return hsum8(T);
}

/* DotF32, kernels.go:37-49 with dotF32AVX2 (kernels_amd64.s:45-85): 32-element
 * steps into four accumulators, then 8-element steps into Y0, HSUM, then a
 * scalar tail s += a*b. Bit parity unpinned (lane order from asm). */
float mref_dot_f32(const float *a, const float *b, int64_t n) {
    if (n < 8) {
        /* dotF32Go, kernels.go:51-66 */
        float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int64_t i = 0;
        for (; i + 4 <= n; i += 4) {
            s0 += a[i] * b[i];
            s1 += a[i + 1] * b[i + 1];
            s2 += a[i + 2] * b[i + 2];
            s3 += a[i + 3] * b[i + 3];
        }
        for (; i < n; i++) s0 += a[i] * b[i];
        return (s0 + s1) + (s2 + s3);
    }
    float Y[4][8] = {{0}};
    int64_t m = n & ~(int64_t)7, i = 0;
    for (; i + 32 <= m; i += 32)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 8; l++) Y[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], Y[r][l]);
    for (; i + 8 <= m; i += 8)
        for (int l = 0; l < 8; l++) Y[0][l] = fmaf(a[i + l], b[i + l], Y[0][l]);
    float s = hsum32(Y);
    for (i = m; i < n; i++) s += a[i] * b[i];
    return s;
}

/* dotQ4KAVX2, kernels_amd64.s:112-170 (tab from q4kScales, kernels.go:209-221):
 * w = f32(d*sc)*q - f32(dmin*m) as the decoder, then fma into the lanes:
 * chunk c elements 64c+{0-7,16-23} -> Y0, {32-39,48-55} -> Y1,
 * {8-15,24-31} -> Y2, {40-47,56-63} -> Y3, then HSUM. Bit parity unpinned. */
float mref_dot_q4k_f32(const uint8_t *row, const float *x, int64_t nb) {
    float Y[4][8] = {{0}};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 144 * b;
        float d = mref_f16_to_f32(le16(blk)), dmin = mref_f16_to_f32(le16(blk + 2));
        const float *xb = x + 256 * b;
        for (int c = 0; c < 4; c++) {
            uint8_t sc0, m0, sc1, m1;
            scale_min_k4(2 * c, blk + 4, &sc0, &m0);
            scale_min_k4(2 * c + 1, blk + 4, &sc1, &m1);
            float s0 = d * (float)sc0, o0 = dmin * (float)m0;
            float s1 = d * (float)sc1, o1 = dmin * (float)m1;
            const uint8_t *q = blk + 16 + 32 * c;
            for (int st = 0; st < 4; st++) { /* Q4STEP at byte offset 8*st */
                int ra = (st & 1) ? 2 : 0, rb = ra + 1;
                for (int l = 0; l < 8; l++) {
                    int i = 8 * st + l;
                    float wl = s0 * (float)(q[i] & 15) - o0;
                    float wh = s1 * (float)(q[i] >> 4) - o1;
                    Y[ra][l] = fmaf(wl, xb[64 * c + i], Y[ra][l]);
                    Y[rb][l] = fmaf(wh, xb[64 * c + 32 + i], Y[rb][l]);
                }
            }
        }
    }
    return hsum32(Y);
}

/* dotQ6KAVX2, kernels_amd64.s:172-282: w = f32(d*sc)*(q-32); part p of each
 * half goes to Y_p, lane l taking l, 8+l, 16+l, 24+l in turn; then HSUM.
 * Bit parity unpinned. */
float mref_dot_q6k_f32(const uint8_t *row, const float *x, int64_t nb) {
    float Y[4][8] = {{0}};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 210 * b;
        float d = mref_f16_to_f32(le16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float *xb = x + 256 * b;
        for (int h = 0; h < 2; h++)
            for (int st = 0; st < 4; st++) /* Q6STEP for l = 8st..8st+7 */
                for (int p = 0; p < 4; p++) {
                    float s = d * (float)sc[8 * h + (st >= 2) + 2 * p];
                    for (int ln = 0; ln < 8; ln++) {
                        int l = 8 * st + ln;
                        float w = s * (float)q6_quant(blk, h, p, l);
                        Y[p][ln] = fmaf(w, xb[128 * h + 32 * p + l], Y[p][ln]);
                    }
                }
    }
    return hsum32(Y);
}

/* dotQ8_0AVX2, kernels_amd64.s:284-308: w = d*q, elements 8r..8r+7 -> Y_r. */
float mref_dot_q8_0_f32(const uint8_t *row, const float *x, int64_t nb) {
    float Y[4][8] = {{0}};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + 34 * b;
        float d = mref_f16_to_f32(le16(blk));
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 8; l++) {
                float w = d * (float)(int8_t)blk[2 + 8 * r + l];
                Y[r][l] = fmaf(w, x[32 * b + 8 * r + l], Y[r][l]);
            }
    }
    return hsum32(Y);
}

/* ------------------------------------------------------------- drivers */

/* RowDot.Load/Dot, kernels.go:122-204: the fused kernel when the row is used
 * at most DecodeOnce = 8 times, else decode once and DotF32. */
static float row_dot_f32(uint32_t dt, const uint8_t *row, const float *x, int64_t k, int fused,
                         const float *decoded) {
    if (!fused) return mref_dot_f32(x, decoded, k);
    switch (dt) {
    case MREF_Q4_K: return mref_dot_q4k_f32(row, x, k / 256);
    case MREF_Q6_K: return mref_dot_q6k_f32(row, x, k / 256);
    case MREF_Q8_0: return mref_dot_q8_0_f32(row, x, k / 32);
    }
    return mref_dot_f32(x, decoded, k);
}

static int fused_q8_blocks(uint32_t dt, int block) {
    /* FusedQ8Blocks, q8.go:105-117, on an AVX2+F16C machine */
    if (block == 32) return dt == MREF_Q4_K || dt == MREF_Q6_K || dt == MREF_Q8_0;
    if (block == 256) return dt == MREF_Q4_K || dt == MREF_Q6_K;
    return 0;
}

/* linearF32/linearCols, fast.go:161-183: y[i*n+j] = Dot(x_i, w_j) (+ bias[j]). */
int mref_linear_f32(const float *x, int64_t rows, const uint8_t *w, uint32_t dt, int64_t n,
                    int64_t k, const float *bias, float *y, int threads) {
    int64_t rb = mref_row_bytes(dt, k);
    if (rb < 0 || dt == MREF_F32 || rows < 0 || n < 0) return MREF_ERR_ARG;
    int fused = rows <= 8 && k > 0;
    (void)threads;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *buf = fused ? NULL : (float *)malloc((size_t)(k > 0 ? k : 1) * 4);
#pragma omp for schedule(static)
        for (int64_t j = 0; j < n; j++) {
            const uint8_t *row = w + rb * j;
            if (!fused) mref_dequantize(dt, row, rb, buf, k);
            for (int64_t i = 0; i < rows; i++) {
                float s = row_dot_f32(dt, row, x + k * i, k, fused, buf);
                if (bias) s += bias[j];
                y[n * i + j] = s;
            }
        }
        free(buf);
    }
    return MREF_OK;
}

/* linearA8, fast.go:282-379 (with dequantMatmulA8, fast.go:246-273): rows of x
 * are quantized to blocks of `block`; a row of x the quantizer refuses, and a
 * row of w with a non-finite block scale, use the float32 path (Load with
 * uses = rows) for all its products; bias added as s + bias[j]. */
int mref_linear_a8(const float *x, int64_t rows, const uint8_t *w, uint32_t dt, int64_t n,
                   int64_t k, const float *bias, int block, float *y, int threads) {
    if (block != 32 && block != 256) return MREF_ERR_ARG;
    int64_t rb = mref_row_bytes(dt, k);
    if (rb < 0 || dt == MREF_F32 || rows < 0 || n < 0) return MREF_ERR_ARG;
    if (!fused_q8_blocks(dt, block)) return mref_linear_f32(x, rows, w, dt, n, k, bias, y, threads);
    if (k % block) return MREF_ERR_ARG;
    int64_t r32 = k / 32;
    int8_t *q = (int8_t *)malloc((size_t)(rows * k + 1));
    float *d = (float *)malloc((size_t)(rows * r32 + 1) * 4);
    float *dbs = (float *)malloc((size_t)(rows * r32 + 1) * 4);
    int16_t *xs = (int16_t *)malloc((size_t)(rows * r32 + 1) * 2);
    int16_t *m32 = (int16_t *)malloc((size_t)(rows * k / 2 + 1) * 2);
    char *ok = (char *)malloc((size_t)rows + 1);
    for (int64_t i = 0; i < rows; i++)
        ok[i] = (char)mref_quantize_act(x + k * i, k, block, q + k * i, d + r32 * i, xs + r32 * i,
                                        m32 + k / 2 * i, dbs + r32 * i);
    int fused = rows <= 8 && k > 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *buf = NULL;
#pragma omp for schedule(static)
        for (int64_t j = 0; j < n; j++) {
            const uint8_t *row = w + rb * j;
            int q8 = 1, decoded = 0;
            for (int64_t i = 0; i < rows; i++) {
                float s = 0;
                int done = 0;
                if (q8 && ok[i]) {
                    if (block == 256)
                        done = dt == MREF_Q4_K
                                   ? mref_dot_q4k_a8k(row, q + k * i, d + r32 * i, xs + r32 * i, k / 256, &s)
                                   : mref_dot_q6k_a8k(row, q + k * i, d + r32 * i, k / 256, &s);
                    else if (dt == MREF_Q4_K)
                        done = mref_dot_q4k_a8(row, q + k * i, d + r32 * i, dbs + r32 * i, k / 256, &s);
                    else if (dt == MREF_Q6_K)
                        done = mref_dot_q6k_a8(row, q + k * i, d + r32 * i, m32 + k / 2 * i, k / 256, &s);
                    else
                        done = mref_dot_q8_0_a8(row, q + k * i, d + r32 * i, k / 32, &s);
                    q8 = done;
                }
                if (!done) {
                    if (!fused && !decoded) {
                        if (!buf) buf = (float *)malloc((size_t)k * 4);
                        mref_dequantize(dt, row, rb, buf, k);
                        decoded = 1;
                    }
                    s = row_dot_f32(dt, row, x + k * i, k, fused, buf);
                }
                if (bias) s += bias[j];
                y[n * i + j] = s;
            }
        }
        free(buf);
    }
    free(q);
    free(d);
    free(dbs);
    free(xs);
    free(m32);
    free(ok);
    return MREF_OK;
}

/* ---- the decoder ops around the linears ---------------------------------
 * Restated from the reference's attention and swiglu fast paths
 * (interp/fast.go:487-498, 559-751; internal/kernels/attn.go:24-140) with
 * the AVX2 kernels they call on amd64 (attn_amd64.s:12-535): the float32
 * operation order is the one of those kernels, so a GPU kernel following
 * the same order gives the same bits. Parity: pinned by the reference
 * fixtures' expected logits (cmd/mim-run/main_test.go tolerances) and by the
 * checks of tests/test_oracle_decoder.py (closed forms, float64 brute
 * force, planted mistakes); the AVX2 bits themselves cannot be run here. */

/* Cephes' expf as expSumF32AVX2 evaluates it (attn_amd64.s:81-240): t is
 * clamped to lo, t = f*ln2 + r with f = rint(t*log2e) and ln2 in two parts,
 * exp(r) = 1 + r + r^2 P(r), times 2^f built in the exponent; t < lo (and
 * NaN) gives 0. */
static inline float cephes_exp_avx2(float t) {
    const float lo = bits_f32(0xc2aeac4fu), log2e = bits_f32(0x3fb8aa3bu);
    const float c1 = bits_f32(0x3f318000u), c2 = bits_f32(0xb95e8083u);
    const int keep = t >= lo;          /* VCMPPS GE_OQ: false for NaN */
    const float tt = t > lo ? t : lo;  /* VMAXPS: the second operand (lo) for NaN */
    const float f = rintf(tt * log2e);
    float r = fmaf(-f, c1, tt);
    r = fmaf(-f, c2, r);
    const float r2 = r * r;
    float p = bits_f32(0x39506967u);
    p = fmaf(p, r, bits_f32(0x3ab743ceu));
    p = fmaf(p, r, bits_f32(0x3c088908u));
    p = fmaf(p, r, bits_f32(0x3d2aa9c1u));
    p = fmaf(p, r, bits_f32(0x3e2aaaaau));
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    const float two_f = bits_f32((uint32_t)((int32_t)f + 127) << 23);
    const float e = p * two_f;
    return keep ? e : 0.0f;
}

/* ExpSumF32 (attn.go:41-56): the first n&~7 through expSumF32AVX2 (eight
 * lane sums, HSUM ((s0+s4)+(s1+s5))+((s2+s6)+(s3+s7))), the rest
 * f32(exp(f64(x-m))) added in order. x[i] becomes its exponential. */
float mref_expsum_f32(float *x, int64_t n, float m) {
    float s = 0.0f;
    int64_t i = 0;
    if (n >= 8) {
        const int64_t nv = n & ~(int64_t)7;
        float lane[8] = {0};
        for (; i < nv; i += 8)
            for (int c = 0; c < 8; c++) {
                const float e = cephes_exp_avx2(x[i + c] - m);
                x[i + c] = e;
                lane[c] = lane[c] + e;
            }
        s = ((lane[0] + lane[4]) + (lane[1] + lane[5])) + ((lane[2] + lane[6]) + (lane[3] + lane[7]));
    }
    for (; i < n; i++) {
        const float e = (float)exp((double)(x[i] - m));
        x[i] = e;
        s += e;
    }
    return s;
}

static inline float kv_val(const float *f32, const uint16_t *f16, int64_t i) {
    return f16 ? mref_f16_to_f32(f16[i]) : f32[i];
}

/* ScoresF32/ScoresF16 with scoresF32AVX2/scoresF16AVX2 (attn_amd64.s:12-78,
 * 312-385), D a multiple of 8: lane c of a row accumulates q[8m+c]*k[8m+c]
 * by fma over m. Rows go in fours from the first, reduced as
 * ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)); the last n%4 rows one by one, as
 * ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)); then times scale. */
void mref_scores(const float *q, const float *k32, const uint16_t *k16, int64_t n, int d, float scale,
                 float *out) {
    const int64_t n4 = n - n % 4;
    for (int64_t j = 0; j < n; j++) {
        float l[8] = {0};
        for (int m = 0; m < d / 8; m++)
            for (int c = 0; c < 8; c++) l[c] = fmaf(q[8 * m + c], kv_val(k32, k16, j * d + 8 * m + c), l[c]);
        const float s = j < n4 ? ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]))
                               : ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
        out[j] = s * scale;
    }
}

/* attendRow (fast.go:728-751) over n visible rows of k and v (f32, or f16
 * when k16/v16 are given), D a multiple of 8: scores, their max, ExpSumF32,
 * WeightedSum (wsumF32AVX2/wsumF16AVX2, attn_amd64.s:244-307, 390-468: per
 * element acc = fma(e_j, v_j, acc) over the rows in order), o = acc / sum.
 * When the largest score is not finite the reference leaves the row to its
 * scalar loop, whose result is then NaN throughout; this restatement writes
 * NaN. sc holds n floats of scratch. */
void mref_attend_row(const float *q, const float *k32, const uint16_t *k16, const float *v32, const uint16_t *v16,
                     int64_t n, int d, float scale, float *sc, float *o) {
    mref_scores(q, k32, k16, n, d, scale, sc);
    float mx = -INFINITY;
    for (int64_t j = 0; j < n; j++)
        if (sc[j] > mx || sc[j] != sc[j]) mx = sc[j];
    if (n == 0 || isinf(mx) || mx != mx) {
        for (int i = 0; i < d; i++) o[i] = n == 0 ? 0.0f : NAN;
        return;
    }
    const float sum = mref_expsum_f32(sc, n, mx);
    for (int i = 0; i < d; i++) {
        float acc = 0.0f;
        for (int64_t j = 0; j < n; j++) acc = fmaf(sc[j], kv_val(v32, v16, j * d + i), acc);
        o[i] = acc / sum;
    }
}

/* The attention of a decoder step over a cache [kv_heads][context][d]
 * (f32, or f16 bits when f16): query t of head h sees the entries
 * kstart[t]..kend[t] of kv head h / (heads / kv_heads). q, out [T][heads][d]. */
int mref_attention(const float *q, const void *kc, const void *vc, const int64_t *kend, const int64_t *kstart,
                   int64_t T, int heads, int kv_heads, int d, int64_t context, int f16, float *out, int threads) {
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || d <= 0 || d % 8) return MREF_ERR_ARG;
    const float scale = (float)(1.0 / sqrt((double)d));
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1) if (threads > 1)
#endif
    for (int64_t th = 0; th < T * heads; th++) {
        const int64_t t = th / heads;
        const int h = (int)(th % heads), hk = h / (heads / kv_heads);
        int64_t k0 = kstart ? kstart[t] : 0;
        if (k0 < 0) k0 = 0;
        if (k0 >= context) k0 = context - 1;
        int64_t n = kend[t] + 1 - k0;
        if (n > context - k0) n = context - k0;
        if (n < 0) n = 0;
        const int64_t base = ((int64_t)hk * context + k0) * d;
        float *sc = (float *)malloc((size_t)(n > 0 ? n : 1) * 4);
        mref_attend_row(q + th * d, f16 ? NULL : (const float *)kc + base, f16 ? (const uint16_t *)kc + base : NULL,
                        f16 ? NULL : (const float *)vc + base, f16 ? (const uint16_t *)vc + base : NULL, n, d, scale,
                        sc, out + th * d);
        free(sc);
    }
    return MREF_OK;
}

/* silu(x) * b as siluMulF32AVX2 computes it (attn_amd64.s:459-535):
 * h = exp(-|x|/2) by the Cephes steps above, e = h*h, silu = x / (1+e) for
 * x >= 0 and ((x*h)*h) / (1+e) below, then times b. */
static inline float silu_mul_avx2(float x, float b) {
    const float t = -fabsf(x) * 0.5f;
    const float h = cephes_exp_avx2(t);
    const float e1 = h * h + 1.0f;
    const float y = (x * h) * h;
    const float num = x >= 0.0f ? x : y;
    return (num / e1) * b;
}

/* swiglu.v1 (fast.go:487-498): parallel() splits the n elements into pieces
 * of max(1, n / (w*8)), w = min(procs, n) (interp/pool.go:33-51, 79-97; one
 * piece when w <= 1), and SiluMulF32 (attn.go:63-76) runs on each piece:
 * its first len&~7 elements through siluMulF32AVX2 (when len >= 8), the
 * rest as f32(f64(a)/(1+exp(-f64(a)))*f64(b)). So the result depends on
 * the reference's GOMAXPROCS, given here as procs. */
void mref_silu_mul(const float *a, const float *b, float *out, int64_t n, int procs) {
    const int64_t w = procs < n ? procs : n;
    int64_t chunk = n;
    if (w > 1) {
        chunk = n / (w * 8);
        if (chunk < 1) chunk = 1;
    }
    for (int64_t lo = 0; lo < n; lo += chunk) {
        const int64_t len = lo + chunk < n ? chunk : n - lo;
        const int64_t nv = len >= 8 ? len & ~(int64_t)7 : 0;
        for (int64_t i = 0; i < len; i++) {
            const float x = a[lo + i], y = b[lo + i];
            out[lo + i] = i < nv ? silu_mul_avx2(x, y)
                                 : (float)((double)x / (1.0 + exp(-(double)x)) * (double)y);
        }
    }
}
