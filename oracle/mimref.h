/*
 * mimref — CPU restatement of the reference numerics of mimir-model's
 * block-quantized linear-layer path (decoders, activation quantizer,
 * block-256 and block-32 8-bit dot products, float32 fused dot products in
 * the AVX2 lane order, and the linearA8/linearF32 drivers).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP
 * library (libmimg.so): only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product path never calls
 * it and has no CPU fallback.
 *
 * Parity status of each function (what pins it) is stated next to its
 * definition in mimref.c.
 */
#ifndef MIMREF_H
#define MIMREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids, as dtype.go:22-46 */
enum {
    MREF_F32 = 1,
    MREF_Q8_0 = 64,
    MREF_Q4_K = 66,
    MREF_Q6_K = 67,
};

/* status codes */
enum {
    MREF_OK = 0,
    MREF_ERR_SIZE = -1,   /* CodeSizeMismatch */
    MREF_ERR_DTYPE = -2,  /* CodeUnsupportedDType / CodeBadDType */
    MREF_ERR_ARG = -3,
};

float mref_f16_to_f32(uint16_t h);
void mref_f16_to_f32_n(const uint16_t *h, float *out, int64_t n);
uint16_t mref_f32_to_f16(float f);

int64_t mref_block_elems(uint32_t dt);
int64_t mref_block_bytes(uint32_t dt);
int64_t mref_row_bytes(uint32_t dt, int64_t k);

int mref_dequantize(uint32_t dt, const uint8_t *src, int64_t src_len, float *dst, int64_t n);
int mref_quantize(uint32_t dt, const float *src, int64_t n, uint8_t *dst, int64_t dst_len);

/* 8-bit activations (q8.go:50-97). Arrays are sized k, k/32, k/32, k/2, k/32.
 * Returns 1 when the row was quantized, 0 when it is refused. */
int mref_quantize_act(const float *x, int64_t k, int block, int8_t *q, float *d,
                      int16_t *xs, int16_t *m32, float *dbs);

/* dot products; each returns 1 and sets *out, or 0 (refused) */
int mref_dot_q4k_a8k(const uint8_t *row, const int8_t *q, const float *d, const int16_t *xs,
                     int64_t nb, float *out);
int mref_dot_q6k_a8k(const uint8_t *row, const int8_t *q, const float *d, int64_t nb, float *out);
int mref_dot_q8_0_a8(const uint8_t *row, const int8_t *q, const float *d, int64_t nb, float *out);
int mref_dot_q4k_a8(const uint8_t *row, const int8_t *q, const float *d, const float *dbs,
                    int64_t nb, float *out);
int mref_dot_q6k_a8(const uint8_t *row, const int8_t *q, const float *d, const int16_t *m32,
                    int64_t nb, float *out);

float mref_dot_f32(const float *a, const float *b, int64_t n);
float mref_dot_q4k_f32(const uint8_t *row, const float *x, int64_t nb);
float mref_dot_q6k_f32(const uint8_t *row, const float *x, int64_t nb);
float mref_dot_q8_0_f32(const uint8_t *row, const float *x, int64_t nb);

/* drivers: fast.go linearA8 / linearF32 (y is rows x n, row-major) */
int mref_linear_a8(const float *x, int64_t rows, const uint8_t *w, uint32_t dt, int64_t n,
                   int64_t k, const float *bias, int block, float *y, int threads);
int mref_linear_f32(const float *x, int64_t rows, const uint8_t *w, uint32_t dt, int64_t n,
                    int64_t k, const float *bias, float *y, int threads);

/* decoder ops (interp/fast.go:487-498, 559-751 with attn_amd64.s) */
float mref_expsum_f32(float *x, int64_t n, float m);
void mref_scores(const float *q, const float *k32, const uint16_t *k16, int64_t n, int d, float scale,
                 float *out);
void mref_attend_row(const float *q, const float *k32, const uint16_t *k16, const float *v32, const uint16_t *v16,
                     int64_t n, int d, float scale, float *sc, float *o);
int mref_attention(const float *q, const void *kc, const void *vc, const int64_t *kend, const int64_t *kstart,
                   int64_t T, int heads, int kv_heads, int d, int64_t context, int f16, float *out, int threads);
void mref_silu_mul(const float *a, const float *b, float *out, int64_t n, int procs);

/* exact fused-multiply-add check helper (fma of floats, for tests) */
float mref_fmaf(float a, float b, float c);

#ifdef __cplusplus
}
#endif
#endif
