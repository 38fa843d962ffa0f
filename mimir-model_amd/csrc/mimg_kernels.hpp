// Kernel launchers of libmimg (host-side declarations shared by the .hip
// files and the C-ABI in mimg_api.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mimg {

// Quantized activations of `rows` rows of K elements, in device memory
// (reference Q8Batch, internal/kernels/q8.go:154-193, with the per-16 sums
// added): q int8 [rows][K]; d32, dbs float [rows][K/32]; xs int16
// [rows][K/32]; ys16 int16 [rows][K/16]; ok int32 [rows].
struct ActPtrs {
    int8_t* q;
    float* d32;
    int16_t* xs;
    int16_t* ys16;
    float* dbs;
    int32_t* ok;
};

// Byte offsets of the ActPtrs arrays in one workspace, each 256-aligned.
struct ActLayout {
    size_t q, d32, xs, ys16, dbs, ok, total;
};
ActLayout act_layout(int64_t rows, int64_t K);
ActPtrs act_ptrs(void* base, const ActLayout& l);

// A registered weight matrix on the device (bytes exactly as in the file).
struct DevWeight {
    uint32_t dt;
    int64_t n, k, row_bytes;
    const uint8_t* data;   // n*row_bytes bytes + WEIGHT_PAD
    const uint8_t* wref;   // n flags: 1 if a block scale of the row is not finite
    int64_t n_refused;
};

hipError_t launch_quantize_act(const float* x, int64_t rows, int64_t K, int block, const ActPtrs& a,
                               hipStream_t stream);
// The producer of a quantized row fused into the quantizer (quantize_act.hip).
struct QaSource {
    const float* aux = nullptr;    // rms_norm: the residual (or null); swiglu: u
    const float* scale = nullptr;  // rms_norm: the scale (or null)
    float eps = 0.f;
    float* y = nullptr;            // the produced rows
    int64_t chunk = 1, total = 0;  // swiglu: the reference's piece size, rows*K
};
hipError_t launch_norm_quantize_act(float* x, const float* resid, const float* scale, float eps, float* y,
                                    int64_t rows, int64_t K, int block, const ActPtrs& a, hipStream_t stream);
hipError_t launch_swiglu_quantize_act(const float* g, const float* u, float* y, int64_t chunk, int64_t rows,
                                      int64_t K, int block, const ActPtrs& a, hipStream_t stream);
hipError_t launch_rope_kv(float* q, const float* k, const float* v, const int64_t* pos, const int64_t* cidx,
                          const double* inv_freq, int T, int H, int Hkv, int D, int rotary, int interleaved, int64_t C,
                          void* kc, void* vc, int f16, hipStream_t s);

hipError_t launch_weight_refusals(uint32_t dt, const uint8_t* w, int64_t n, int64_t k, uint8_t* wref,
                                  hipStream_t stream);

// y_i[r*N_i+j] for act rows r in [0, rows) of up to three matrices of one
// dtype and K (rows <= 8 per launch; `total_rows` is the row count of the
// whole call, which selects the float32 fallback's order).
// The decode GEMV for 2..8 activation rows on the int8 matrix cores
// (gemv_mfma.hip): same arguments and results as launch_gemv_a8k.
bool gemv_mfma_ok(const DevWeight* const* ws, int nmat, int64_t rows);
hipError_t launch_gemv_a8k_mfma(const DevWeight* const* ws, int nmat, const ActPtrs& a, int64_t rows,
                                int64_t total_rows, const float* x, const float* const* bias, float* const* y,
                                hipStream_t stream);
// gate and up (Q4_K, same shape) at one pre-quantized row with swiglu.v1
// in the epilogue: out[n] = swiglu(gate[n], up[n]) with the reference's
// pieces of `chunk` elements of `total` (gemv_kquant.hip).
bool gemv_swiglu_ok(const DevWeight& gate, const DevWeight& up);
bool gemv_mfma_swiglu_ok(const DevWeight& gate, const DevWeight& up, int64_t rows);
hipError_t launch_gemv_a8k_mfma_swiglu(const DevWeight& gate, const DevWeight& up, const ActPtrs& a, int64_t rows,
                                       const float* x, const float* const* bias, float* out, int64_t total,
                                       int64_t chunk, hipStream_t stream);
hipError_t launch_gemv_a8k_swiglu(const DevWeight& gate, const DevWeight& up, const ActPtrs& a, const float* x,
                                  const float* const* bias, float* out, int64_t total, int64_t chunk,
                                  hipStream_t stream);
hipError_t launch_gemv_a8k(const DevWeight* const* ws, int nmat, const ActPtrs& a, int64_t rows,
                           int64_t total_rows, const float* x, const float* const* bias, float* const* y,
                           hipStream_t stream);

// Independent one-row products in one launch (gemv_kquant.hip): segment i
// is matrix W (Q4_K or Q6_K, K a multiple of 256) against its own quantized
// row; the launcher orders the segments and sets tile0.
struct SetSeg {
    const uint8_t* W;
    const uint8_t* wref;
    const float* bias;    // [N] or null
    float* y;             // [N]
    const int8_t* q;      // the segment's quantized row
    const float* d32;
    const int16_t* s16;   // Q4_K: xs; Q6_K: ys16
    const int32_t* ok;
    const float* x;       // the f32 row (float32 path of refused rows)
    int64_t rb, K;
    int32_t N, nb, dt, pad;
};
constexpr int SET_MAXSEG = 16;
struct SetArgs {
    int32_t tile0[SET_MAXSEG];  // first workgroup of each segment (INT_MAX past nseg)
    int32_t nseg, pad[3];
    SetSeg seg[SET_MAXSEG];
};
hipError_t launch_gemv_a8k_set(const SetArgs& a, hipStream_t stream);
// One launch quantizing rows of different K (blocks of 256; each row's own
// ActPtrs), as launch_quantize_act on each (quantize_act.hip).
struct QaSetRow {
    const float* x;
    int64_t K;
    ActPtrs a;
    int32_t wg0, pad;  // first workgroup: the row's scanner, then its chunk workgroups
};
constexpr int QA_SET_MAXROWS = 16;
struct QaSetArgs {
    QaSetRow row[QA_SET_MAXROWS];
    int32_t nrows, pad[3];
};
hipError_t launch_quantize_act_set(const QaSetArgs& a, int wgs, hipStream_t stream);

// Many activation rows (already quantized) against one Q4_K/Q6_K matrix,
// on the int8 matrix cores (gemm_kquant.hip); bit-identical to the GEMV.
bool gemm_a8k_ok(const DevWeight& w);
// The 16 x 16 x 64 form for small grids (gemm_kquant16.hip); launch_gemm_a8k
// picks it by grid size.
hipError_t launch_gemm_a8k_16(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                              const float* bias, float* y, hipStream_t stream);
hipError_t launch_gemm_a8k(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                           const float* bias, float* y, hipStream_t stream);

// One activation row, quantized inside the kernel, against up to three
// Q4_K/Q6_K matrices with the same K (gemv_fused.hip).
bool fused_gemv_ok(const DevWeight* const* ws, int nmat);
hipError_t launch_gemv_a8k_fused(const DevWeight* const* ws, int nmat, const float* x,
                                 const float* const* bias, float* const* y, hipStream_t stream);
// The same with rms_norm.v1 in front: y = rms_norm(x + resid) * scale is
// quantized and multiplied; x + resid is written to x_out (not in place: the
// workgroups all read x). One activation row, K a multiple of 1024, <= 4096.
bool fused_norm_ok(const DevWeight* const* ws, int nmat);
hipError_t launch_gemv_a8k_fused_norm(const DevWeight* const* ws, int nmat, const float* x, const float* resid,
                                      const float* scale, float eps, float* x_out, const float* const* bias,
                                      float* const* y, hipStream_t stream);
// q and k (rope) and v (cache scatter) at 2..8 activation rows on the
// matrix cores (gemv_mfma.hip), as the separate products and rope_kv.
bool gemv_mfma_qkv_ok(const DevWeight* const* ws, int64_t rows, int heads, int kv_heads, int d, int rotary);
hipError_t launch_gemv_a8k_mfma_qkv(const DevWeight* const* ws, const ActPtrs& a, int64_t rows, const float* x,
                                    const float* const* bias, float* q, const int64_t* pos, const int64_t* cidx,
                                    const double* inv_freq, int heads, int kv_heads, int d, int rotary,
                                    int interleaved, int64_t context, void* kc, void* vc, int f16,
                                    hipStream_t stream);
// The rope.v1 + cache scatter epilogue of the fused q/k/v GEMV at one row.
struct FusedRope {
    const int64_t* pos;
    const int64_t* cidx;
    const double* inv_freq;
    int heads, kv_heads, d, rotary, interleaved, f16;
    int64_t context;
    void* kcache;
    void* vcache;
};
bool fused_norm_rope_ok(const DevWeight* const* ws, int heads, int kv_heads, int d, int rotary);
hipError_t launch_gemv_a8k_fused_norm_rope(const DevWeight* const* ws, const float* x, const float* resid,
                                           const float* scale, float eps, float* x_out, const float* const* bias,
                                           float* q, const FusedRope& rope, hipStream_t stream);

// Many activation rows (quantized in blocks of 32) against one Q8_0 matrix
// with K a multiple of 256, on the int8 matrix cores (gemm_q8_0.hip): exact
// block sums, one float chain in block order (within the spec's tolerance).
bool gemm_q8_0_ok(const DevWeight& w);
// Q4_K / Q6_K x activations in blocks of 32 on the int8 matrix cores (one
// float chain of exact block sums: a tolerance claim, gemm_kq_b32.hip).
bool gemm_kq_b32_ok(const DevWeight& w);
// The small-grid tiling of both (16 weight rows x 64 activation rows, four
// waves; gemm_b32s.hip): the same per-output arithmetic.
int64_t gemm_b32_small_wgs(int64_t n, int64_t rows);
hipError_t launch_gemm_b32_small(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows,
                                 const float* x, const float* bias, float* y, hipStream_t stream);
hipError_t launch_gemm_kq_b32(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                              const float* bias, float* y, hipStream_t stream);
hipError_t launch_gemm_q8_0(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows, const float* x,
                            const float* bias, float* y, hipStream_t stream);

hipError_t launch_gemv_q8_0_a8(const DevWeight& w, const ActPtrs& a, int64_t rows,
                               int64_t total_rows, const float* x, const float* bias, float* y,
                               int64_t y_stride, hipStream_t stream);

// Q4_K/Q6_K x 8-bit activations in blocks of 32, rows <= 8 per launch
// (gemv_kquant_b32.hip).
hipError_t launch_gemv_kq_a8_b32(const DevWeight& w, const ActPtrs& a, int64_t rows, int64_t total_rows,
                                 const float* x, const float* bias, float* y, int64_t y_stride,
                                 hipStream_t stream);

hipError_t launch_linear_f32(const DevWeight& w, const float* x, int64_t rows, const float* bias,
                             float* y, hipStream_t stream);
// The same product on the fp32 matrix cores, within the spec's bound for
// dequant_matmul.v1 (gemm_f32.hip).
hipError_t launch_linear_f32_mfma(const DevWeight& w, const float* x, int64_t rows, const float* bias, float* y,
                                  hipStream_t stream);

// Decoder-step ops (decoder_ops.hip).
hipError_t launch_embed_rows(uint32_t dt, const uint8_t* table, int64_t row_bytes, const int32_t* ids, int T, int V,
                             int64_t E, float* out, hipStream_t s);
hipError_t launch_rms_norm(float* x, const float* resid, const float* scale, float eps, int64_t rows, int64_t n, float* y,
                           hipStream_t s);
hipError_t launch_rope(float* x, const int64_t* pos, const double* inv_freq, int T, int heads, int D, int rotary,
                       int interleaved, hipStream_t s);
hipError_t launch_kv_store(const float* k, const float* v, const int64_t* pos, int T, int Hkv, int D, int64_t C, void* kc,
                           void* vc, int f16, hipStream_t s);
hipError_t launch_attention(const float* q, const void* kc, const void* vc, const int64_t* kend, const int64_t* kstart,
                            int T, int H, int Hkv, int D, int64_t C, int64_t maxk, int f16, float* out, float* ws,
                            hipStream_t s);
hipError_t launch_greedy_advance(const int32_t* chosen, int32_t* ids, int64_t* pos, int64_t* cidx, int32_t* out,
                                 int32_t* count, int cap, int n, hipStream_t s);
hipError_t launch_swiglu(const float* g, const float* u, float* out, int64_t n, int64_t chunk, hipStream_t s);
hipError_t launch_argmax(const float* x, int64_t rows, int64_t n, int32_t* out, hipStream_t s);

hipError_t launch_dequantize(uint32_t dt, const uint8_t* src, int64_t n_elems, float* dst,
                             hipStream_t stream);

hipError_t launch_encode(uint32_t dt, const float* x, int64_t n, uint8_t* dst, hipStream_t stream);

// A plain streaming read of up to eight byte ranges (misc_kernels.hip), the
// measured ceiling of the HBM-bound kernels; per = 16-byte loads per thread
// (2, 4, 8 or 16), one workgroup of 256 threads per per*4 KB.
constexpr int READ_MAX_RANGES = 8;
struct ReadRanges {
    const uint8_t* src[READ_MAX_RANGES];
    int64_t len[READ_MAX_RANGES];  // multiples of 16
    int64_t wgs[READ_MAX_RANGES];  // workgroups per range (set by the launcher)
    int count;
};
hipError_t launch_stream_read(const ReadRanges& r, int per, uint32_t* sink, hipStream_t s);
hipError_t launch_normal_fill(uint64_t seed, float stdv, float* dst, int64_t n, hipStream_t stream);

// A chain of dependent one-row products in one launch (chain.hip): phase p
// is the grouped 8-bit product (blocks of 256) of up to three Q4_K / Q6_K
// matrices with its input row x; a phase may read rows earlier phases
// wrote. One workgroup per CU, all resident at once (G = the CU count).
constexpr int CHAIN_MAXP = 8;            // phases per launch
constexpr int CHAIN_MAXK = 16384;        // input row length
constexpr int CHAIN_STAGE_BYTES = 16384; // a stage: whole rows, at most this many bytes
constexpr int CHAIN_MAX_PAIRS = 128;     // (row, block) pairs per stage
constexpr int CHAIN_LINES = 16;          // line counters of a device barrier
constexpr int CHAIN_TABLE_ENTRIES = 2560;  // (row, block) pairs of one phase per workgroup
struct ChainMat {
    const uint8_t* W;     // rows of rb bytes (rb a multiple of 16)
    const uint8_t* wref;  // [N] weight-row refusal flags
    const float* bias;    // [N] or null
    float* y;             // [N]
    int32_t N, dt, rb, rps;  // rps: rows per stage
    int32_t nref, pad;    // rows with a refused block scale (0: wref is not read)
};
struct ChainPhase {
    const float* x;       // [K], 16-byte aligned
    int64_t bytes;        // weight bytes of the phase's matrices
    int32_t K, nb, nmat, pad;
    ChainMat m[3];
};
struct ChainArgs {
    ChainPhase ph[CHAIN_MAXP];
    uint64_t* sync;       // status word, then (nphase-1) x (1 + CHAIN_LINES) counters 128 bytes apart
    int32_t nphase, G, lines, pad;
};
constexpr uint64_t CHAIN_SYNC_BYTES = 128ull * (1 + (CHAIN_MAXP - 1) * (1 + CHAIN_LINES));
int chain_occupancy();  // resident chain workgroups per CU
hipError_t launch_chain(const ChainArgs& A, hipStream_t stream);
hipError_t launch_chain_zero(void* p, uint64_t bytes, hipStream_t stream);  // bytes: a multiple of 8

}  // namespace mimg
