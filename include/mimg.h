/*
 * mimg.h — C ABI of libmimg, the MI355X (gfx950) block-quantized
 * linear-layer path of mimir-model.
 *
 * The reference runs these products on the CPU inside the interp executor's
 * fast paths:
 *
 *   type fastFunc func(attrs []mim.Attr, in []*ref.Tensor, dts []mim.DType,
 *                      shapes [][]int) (out []*ref.Tensor, handled bool, err error)
 *   fastPaths["dequant_matmul_a8.v2" | "dequant_matmul_a8.v1" | "dequant_matmul.v1"]
 *                                                  (reference interp/fast.go:40-59)
 *
 * A Go cgo shim (mimir-model_amd/go/mimg_fast.go) registers replacements for
 * those keys that call the functions below; the signature of fastFunc and
 * its callers (interp/interp.go:853-877, interp/plan.go:834-896) are
 * unchanged. Plain pointers and sizes only.
 *
 * Status codes: 0 = done; > 0 = not handled, the caller runs its own path
 * (the reference's handled = false); < 0 = error, text in mimg_last_error().
 * No function aborts the process.
 *
 * Dtype ids are mim's (reference dtype.go:22-46): F32 = 1, Q8_0 = 64,
 * Q4_K = 66, Q6_K = 67. Weights are [N, K] row-major in their on-disk block
 * layout (spec/dtypes.md), uploaded once and never repacked.
 *
 * Thread safety: every function may be called from any thread. Host-memory
 * entry points run on a stream owned by the calling thread and return when
 * the result is in host memory. Device-memory entry points (suffix _dev)
 * enqueue on the caller's stream and return at once; device pointers must
 * stay valid until that stream reaches the work.
 */
#ifndef MIMG_H
#define MIMG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIMG_OK 0
#define MIMG_NOT_HANDLED 1
#define MIMG_ERR_ARG (-1)
#define MIMG_ERR_HIP (-2)
#define MIMG_ERR_NOT_INIT (-3)
#define MIMG_ERR_HANDLE (-4)
#define MIMG_ERR_DEVICE (-5)
#define MIMG_ERR_WORKSPACE (-6)

#define MIMG_DT_F32 1u
#define MIMG_DT_Q8_0 64u
#define MIMG_DT_Q4_K 66u
#define MIMG_DT_Q6_K 67u

/* Selects the GPU and checks that it is gfx950. Idempotent for one device.
 * No reference counterpart: the reference runs on the CPU; a Program's
 * lifetime (interp.Load, interp/interp.go:101-122) brackets init/shutdown. */
int mimg_init(int device);

/* Waits for the device, frees every registered weight (a view's bytes with
 * its section), every uploaded weights section and the calling thread's
 * stream and buffers (other threads' go when those threads exit), and
 * forgets the device, so mimg_init may be called again. A weight that a
 * call on another thread still holds is unlinked instead and freed after
 * that call returns (with its section, for a view), at the next release,
 * registration or shutdown; such a call must not start new work after the
 * shutdown. Synchronises the device and frees memory: not during a graph
 * capture. */
void mimg_shutdown(void);

/* Text of the last error of the calling thread ("" if none). */
const char *mimg_last_error(void);

/* Library version, (major << 16) | minor. */
int mimg_version(void);

/* Uploads a weight matrix once, byte for byte, and returns its handle.
 * Replaces the zero-copy ref.Tensor{Data: f.TensorData(t)} the fast paths
 * read (interp/interp.go:101-122 -> file.go:394-398): the same (host, len,
 * dtype, n, k) returns the same handle without a second upload, so a Go
 * caller may pass W.Data of every call (its mmap slice is stable for the
 * Program's life). A hit is checked against a sampled fingerprint of the
 * bytes (64 samples and both ends), so other bytes later mapped at the same
 * address (a file closed and another opened) are uploaded afresh. Each call
 * adds a reference; mimg_release_weight drops one. len must equal
 * n * (k / block_elems) * block_bytes. */
int mimg_register_weight(const void *host, uint64_t len, uint32_t dtype, int64_t n, int64_t k,
                         uint64_t *handle);

/* As mimg_register_weight for bytes already in device memory (copied into a
 * buffer of the library; no host key). No reference counterpart: for callers
 * that keep the file's weights resident on the GPU. */
int mimg_register_weight_device(const void *dev, uint64_t len, uint32_t dtype, int64_t n, int64_t k,
                                uint64_t *handle);

/* The container's weights section uploaded whole (reference File.Weights(),
 * file.go:401-404; spec/container.md sections 6.3 and 7: one contiguous,
 * aligned byte range): len bytes from host into one device buffer in one
 * transfer, followed by 256 zero bytes; *dev receives its address. Tensors
 * keep their offsets in it, so each weight is a view (below). */
int mimg_upload_weights(const void *host, uint64_t len, void **dev);

/* Frees an uploaded weights section; fails while views of it are registered. */
int mimg_free_weights(void *dev);

/* A weight matrix inside an uploaded weights section, at device address dev
 * (section base + the tensor's offset): as mimg_register_weight, without a
 * copy. Its handle is released with mimg_release_weight. */
int mimg_register_weight_view(const void *dev, uint64_t len, uint32_t dtype, int64_t n, int64_t k,
                              uint64_t *handle);

/* Drops one reference of a registration; the last frees the device buffer
 * (a view's flags only). A call that looked the handle up before the last
 * release keeps the weight alive until it returns, so sessions on several
 * threads may share weights (reference interp/pool.go:30-40,
 * interp/interp.go:409-523 run sessions concurrently); the handle itself
 * is unknown to calls that start after the last release; such a call hands
 * the weight over when it returns, and it is freed at the next release,
 * registration or shutdown (a call may be enqueuing under graph capture,
 * where nothing may be freed). Releases and registrations may synchronise
 * the device and free memory: not during a graph capture. */
int mimg_release_weight(uint64_t handle);

/* Device address of a weight's bytes and the number of its rows that the
 * 8-bit kernels refuse (a block scale that is not finite). */
int mimg_weight_info(uint64_t handle, const void **dev_ptr, int64_t *n_refused);

/* ---- host-memory entry points: one fast-path call each ------------------ */

/* dequant_matmul_a8.v1 (block = 32) and dequant_matmul_a8.v2 (block = 32 or
 * 256): y[rows, N] = x[rows, K] . W^T + bias with x quantized to 8-bit
 * blocks (reference fastDequantMatmulA8/fastDequantMatmulA8V2 ->
 * dequantMatmulA8 -> linearA8, interp/fast.go:226-379; attribute check
 * a8Block, interp/transformer.go:201-214). A dtype without an 8-bit kernel
 * for `block` runs the float32 path, as the reference does (fast.go:256-259).
 * Rows of x with a NaN or |x| > 2^60, and rows of W with a non-finite block
 * scale, use the float32 path (fast.go:323-377). bias may be NULL. Returns
 * MIMG_ERR_ARG for block not in {32, 256} (the reference's error).
 * Order: blocks of 256 are bit for bit the reference (dotQ8KRef); blocks of
 * 32 follow the AVX2 lane order of dotQ8_0Q8AVX2 / dotQ4KQ8AVX2 /
 * dotQ6KQ8AVX2 at every row count, so a row's result never depends on the
 * other rows of the call (mimg_matmul_a8_quantized_q8_0_tiled_dev is the
 * matrix-core form of the Q8_0 product, a tolerance claim a caller opts
 * into). */
int mimg_dequant_matmul_a8(uint64_t w, const float *x, int64_t rows, const float *bias, int block,
                           float *y);

/* dequant_matmul.v1: float32 activations (reference fastDequantMatmul ->
 * linearFast -> linearF32, interp/fast.go:161-224). */
int mimg_dequant_matmul(uint64_t w, const float *x, int64_t rows, const float *bias, float *y);

/* mim.Dequantize for Q8_0, Q4_K and Q6_K, bit for bit (reference
 * quant.go:37-73): src holds len bytes, dst n floats. Errors as the
 * reference: size mismatch -> MIMG_ERR_ARG, other dtypes -> MIMG_NOT_HANDLED. */
int mimg_dequantize(uint32_t dtype, const void *src, uint64_t len, float *dst, int64_t n);

/* ---- device-memory entry points (async on `stream`, a hipStream_t) ------ */

/* Bytes of the workspace the 8-bit entry points need for rows x K. */
uint64_t mimg_a8_workspace_bytes(int64_t rows, int64_t k);

/* Byte offsets, inside that workspace, of the quantized activations:
 * off[0] q int8[rows][K], off[1] d float[rows][K/32], off[2] xs
 * int16[rows][K/32], off[3] ys16 int16[rows][K/16], off[4] dbs
 * float[rows][K/32], off[5] ok int32[rows]. (Reference Q8Batch layout,
 * internal/kernels/q8.go:154-193, with per-16 sums added.) */
int mimg_a8_workspace_offsets(int64_t rows, int64_t k, uint64_t off[6]);

/* Q8.QuantizeBlocks for each row of x (reference internal/kernels/q8.go:50-97)
 * into the workspace. x must be 16-byte aligned. */
int mimg_quantize_act_dev(const float *x, int64_t rows, int64_t k, int block, void *ws,
                          uint64_t ws_bytes, void *stream);

/* mimg_dequant_matmul_a8 on device buffers: quantizes x into ws, then runs
 * the product. y is [rows, N] row-major and must not overlap x (here and in
 * the other product entry points on device buffers: MIMG_ERR_ARG). */
int mimg_linear_a8_dev(uint64_t w, const float *x, int64_t rows, const float *bias, int block, float *y,
                       void *ws, uint64_t ws_bytes, void *stream);

/* mimg_linear_a8_dev for `count` (1..3) weights with the same K that share
 * the activations x, e.g. the q, k and v projections of a decoder layer
 * (reference importer/llama.go:423-534 writes them as three
 * dequant_matmul_a8 calls on one input). y[i] (and bias[i], or bias NULL)
 * belong to weight i. Equal, bit for bit, to the separate calls; with one
 * activation row and blocks of 256 it is a single launch that quantizes x
 * inside the kernel (ws may then be NULL). */
int mimg_linear_a8_group_dev(const uint64_t *w, int count, const float *x, int64_t rows,
                             const float *const *bias, int block, float *const *y, void *ws,
                             uint64_t ws_bytes, void *stream);

/* One phase of mimg_linear_a8_chain_dev: the grouped product of `count`
 * (1..3) weights sharing K on the input row x, as mimg_linear_a8_group_dev
 * with one activation row and blocks of 256. */
typedef struct {
    const float *x;       /* [K], 16-byte aligned */
    int count;
    uint64_t w[3];
    const float *bias[3]; /* each [N_i] or NULL */
    float *y[3];          /* each [N_i] */
} mimg_chain_phase;

/* A chain of 1..8 such phases in one launch, bit for bit the calls
 * mimg_linear_a8_group_dev(phase 0), then phase 1, ... in order: a
 * phase's x may be an output of an earlier phase of the chain (the
 * q/k/v -> o -> gate/up -> down sequence of calls importer/llama.go:423-534
 * writes for one decoder layer, each a dequant_matmul_a8.v2 at
 * interp/fast.go:246-379). The weights of every phase stream from HBM
 * without a break between the phases; a phase waits for the one before it
 * on a device-wide barrier whose counters live in `sync` (at least
 * mimg_chain_sync_bytes(), 256-byte aligned, zeroed once before its first
 * use, e.g. by mimg_chain_sync_init; its counters only grow, so a captured
 * graph of the call can be replayed). Calls that share a sync buffer must
 * not overlap in time. y of a phase must not overlap that phase's x, nor
 * another y of the same phase (MIMG_ERR_ARG). Returns MIMG_NOT_HANDLED
 * (nothing launched) unless every weight is Q4_K or Q6_K with K a multiple
 * of 256 up to 16384, its rows a multiple of 16 bytes (Q6_K: K a multiple
 * of 2048) and at most 16 KB: the caller then makes the group calls.
 * A phase whose barrier wait exceeds its bound (only if the GPU cannot hold
 * every workgroup of the launch at once) finishes without valid outputs and
 * sets the status word that mimg_chain_status reports. */
int mimg_linear_a8_chain_dev(const mimg_chain_phase *phases, int nphase, void *sync, uint64_t sync_bytes,
                             void *stream);
uint64_t mimg_chain_sync_bytes(void);
/* Zeroes a sync buffer on `stream` (a fill kernel, safe under capture). */
int mimg_chain_sync_init(void *sync, uint64_t sync_bytes, void *stream);
/* Reads the status word of a sync buffer into *status (0: every barrier
 * wait completed) and clears it; synchronises with the device. */
int mimg_chain_status(void *sync, uint32_t *status);

/* Independent one-row products in two launches: `ngroups` (1..8) groups,
 * each the grouped product of `count` (1..3) weights sharing K on its own
 * input row x (the mimg_chain_phase fields; at most 16 weights in all), as
 * mimg_linear_a8_group_dev with one activation row and blocks of 256 on each
 * group (interp/fast.go:246-379, dequant_matmul_a8.v2 at block 256), bit for
 * bit. One launch quantizes every group's row into `ws` (at least
 * mimg_linear_a8_set_workspace_bytes, 256-byte aligned), one launch runs all
 * the products, Q4_K and Q6_K mixed, so no product waits for another's
 * launch to drain. For a layer's linears whose inputs do not depend on each
 * other's outputs (BASELINE cfg1's linear set; a decoder layer's own calls
 * are dependent and keep mimg_linear_a8_group_dev). No output may overlap
 * any group's x or another output (MIMG_ERR_ARG). Returns MIMG_NOT_HANDLED
 * (nothing launched) unless every weight is Q4_K or Q6_K with K a multiple
 * of 256 up to 65536. No counterpart in the reference, which runs each
 * product as a call of its own. */
int mimg_linear_a8_set_dev(const mimg_chain_phase *groups, int ngroups, void *ws, uint64_t ws_bytes, void *stream);
int mimg_linear_a8_set_workspace_bytes(const mimg_chain_phase *groups, int ngroups, uint64_t *bytes);
/* The product launch of mimg_linear_a8_set_dev alone, on rows a set call
 * with the same groups already quantized into ws (group g's row at the sum
 * of mimg_a8_workspace_bytes(1, K_h) over the groups h before it; x is
 * still read for the float32 path of refused rows). No counterpart in the
 * reference (its products quantize their own rows). */
int mimg_matmul_a8_quantized_set_dev(const mimg_chain_phase *groups, int ngroups, void *ws, uint64_t ws_bytes,
                                     void *stream);
#define MIMG_SET_MAX_GROUPS 8

/* mimg_linear_a8_dev without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): the quantized activations go to a scratch array
 * of mimg_noalloc_scratch_bytes() (4 MiB) in the library's device memory,
 * one per GPU, kept until the process ends. The call allocates nothing.
 * Rows x K whose workspace (mimg_a8_workspace_bytes) exceeds the scratch
 * return MIMG_ERR_WORKSPACE (e.g. at most ~800 rows at K = 4096, ~230 at
 * K = 14336). Every call on one GPU shares its scratch: calls that overlap
 * in time on that GPU (other streams or threads) race and must be
 * serialised by the caller. No counterpart in the reference. */
int mimg_linear_a8_noalloc_dev(uint64_t w, const float *x, int64_t rows, const float *bias, int block, float *y,
                               void *stream);
uint64_t mimg_noalloc_scratch_bytes(void);

/* rms_norm.v1 in front of mimg_linear_a8_group_dev at one activation row,
 * blocks of 256, in one launch: x_out = x + resid (x copied when resid is
 * NULL), h = rms_norm(x_out) * scale (reference interp/fast.go:434-485), and
 * y[i] = h . W_i^T (+ bias[i]) as dequant_matmul_a8 computes it
 * (interp/builtins.go dequant_matmul_a8.v2, q8.go:50-97). Bit for bit
 * mimg_rms_norm_dev followed by mimg_linear_a8_group_dev. x_out must not
 * overlap x, resid or scale, and no y[i] may overlap x, resid, scale or
 * x_out (every workgroup reads them; MIMG_ERR_ARG). Returns MIMG_NOT_HANDLED
 * (nothing launched) unless K is a multiple of 1024 up to 4096, every
 * weight is Q4_K or Q6_K and the group's rows fit one launch: the caller
 * then makes the two calls. No reference counterpart beyond the two ops it
 * equals (importer/llama.go:423-534 writes the norm and the q, k, v
 * products as separate graph nodes). */
int mimg_rms_norm_linear_a8_group_dev(const uint64_t *w, int count, const float *x, const float *resid,
                                      const float *scale, float eps, float *x_out, const float *const *bias,
                                      float *const *y, void *stream);

/* The gate and up products of the FFN (w = {gate, up}) on 1 to 8 rows of
 * activations already quantized into ws, and swiglu.v1 (reference
 * interp/fast.go:487-498, SiluMulF32 over the pieces of parallel() with
 * GOMAXPROCS = procs, over the flattened [rows, N] products) of the two, in
 * one launch: out[t][n] = swiglu(gate[t][n], up[t][n]), bit for bit
 * mimg_matmul_a8_quantized_group_dev then mimg_swiglu_dev of rows*N
 * elements; the products themselves are not written. bias may be NULL or
 * hold NULLs. Returns MIMG_NOT_HANDLED (nothing launched) unless block is
 * 256, both weights are Q4_K of one shape and N is a multiple of 4 (one
 * row) or 8 (2..8 rows). No reference counterpart beyond the ops it
 * equals. */
int mimg_matmul_a8_quantized_swiglu_dev(const uint64_t *w, const float *x, int64_t rows, const float *const *bias,
                                        int block, float *out, int procs, const void *ws, uint64_t ws_bytes,
                                        void *stream);

/* The q, k, v products (w = {q, k, v}) of 4 to 8 activation rows already
 * quantized into ws (blocks of 256), then rope.v1 on q and k and the cache
 * scatter of k and v at cache_index[t] of each row t (reference
 * interp/fast.go:507-557, importer/llama.go:489-503), in one launch
 * instead of four: bit for bit
 * mimg_matmul_a8_quantized_group_dev then mimg_rope_kv_dev, with q written
 * to q [rows, heads, d] and k and v to the caches only. Returns
 * MIMG_NOT_HANDLED (nothing launched) outside 4..8 rows, block 256, d 64 or
 * 128, q and k of one dtype and q, k, v of heads*d, kv_heads*d, kv_heads*d
 * rows. No reference counterpart beyond the ops it equals. */
int mimg_matmul_a8_quantized_qkv_rope_kv_dev(const uint64_t *w, const float *x, int64_t rows,
                                             const float *const *bias, int block, float *q, const int64_t *pos,
                                             const int64_t *cache_index, const double *inv_freq, int heads,
                                             int kv_heads, int d, int rotary, int interleaved, int64_t context,
                                             void *kcache, void *vcache, int f16, const void *ws, uint64_t ws_bytes,
                                             void *stream);

/* mimg_rms_norm_linear_a8_group_dev on w = {q, k, v} at one activation
 * row followed by mimg_rope_kv_dev (T = 1) on its outputs, in one launch:
 * rope.v1 (reference interp/fast.go:507-557) rotates q (written to q,
 * [heads, d]) and k, and the cache scatter of importer/llama.go:489-503
 * stores the rotated k and v into kcache/vcache at cache_index[0] (not
 * stored outside 0..context-1). Bit for bit the two calls; the k and v
 * outputs are not written anywhere else. q must not overlap x, resid, scale
 * or x_out (MIMG_ERR_ARG). Returns MIMG_NOT_HANDLED (nothing launched)
 * where the fused norm GEMV does not take the shape, where q, k, v are not
 * [heads*d], [kv_heads*d], [kv_heads*d] rows, or where a workgroup's rows
 * would not be whole rotation pairs of one head: the caller then makes the
 * two calls. No reference counterpart beyond the ops it equals. */
int mimg_rms_norm_qkv_rope_kv_dev(const uint64_t *w, const float *x, const float *resid, const float *scale,
                                  float eps, float *x_out, const float *const *bias, float *q, const int64_t *pos,
                                  const int64_t *cache_index, const double *inv_freq, int heads, int kv_heads, int d,
                                  int rotary, int interleaved, int64_t context, void *kcache, void *vcache, int f16,
                                  void *stream);

/* The product alone, for activations already quantized into ws by
 * mimg_quantize_act_dev with the same rows, K and block. */
int mimg_matmul_a8_quantized_dev(uint64_t w, const float *x, int64_t rows, const float *bias, int block,
                                 float *y, const void *ws, uint64_t ws_bytes, void *stream);

/* Q8_0 weights times activations quantized in blocks of 32 (ws from
 * mimg_quantize_act_dev with block 32), on the int8 matrix cores: each
 * output is one float chain over its blocks, tot = fma(f32(S_b),
 * d_b*dx_b, tot) with S_b the exact int32 block sum, then the bias. This is
 * NOT the reference's order (dotQ8_0Q8AVX2, internal/kernels/
 * kernels_amd64.s:1007-1043, keeps eight lane chains), so the results are a
 * tolerance claim: within the spec's dequant_matmul_a8 bound
 * (spec/stdlib.md:260-275) of the exact product. Each row's result depends
 * on that row alone. mimg_linear_a8_dev and the other entry points keep the
 * reference's lane order at every row count; a caller opts into this one.
 * Refused rows (NaN or |x| > 2^60, non-finite weight scales) take the
 * reference-order float32 path. Returns MIMG_NOT_HANDLED for shapes it
 * does not tile. No reference counterpart: a faster form of the products
 * interp/fast.go:282-379 makes, for callers that accept the tolerance. */
int mimg_matmul_a8_quantized_q8_0_tiled_dev(uint64_t w, const float *x, int64_t rows, const float *bias, float *y,
                                            const void *ws, uint64_t ws_bytes, void *stream);

/* The matrix-core products with activation blocks of 32 for Q8_0, Q4_K and
 * Q6_K weights (ws from mimg_quantize_act_dev with block 32): Q8_0 as
 * mimg_matmul_a8_quantized_q8_0_tiled_dev; Q4_K and Q6_K in the reference's
 * per-block form of dotQ4KQ8AVX2 / dotQ6KQ8AVX2 (internal/kernels/
 * kernels_amd64.s:428-597, 760-882) with one float chain where those keep
 * eight lanes: per weight block, over its activation blocks j in order,
 * t = fma(f32(S_j), dx_j, t) with S_j the exact int32 sum of sc * q * y over
 * block j (Q6_K: both sub-blocks of 16 with their scales), tot = fma(d, t,
 * tot); Q4_K also off = fma(dmin * f32(m_j), dbs_j, off); result tot - off
 * (Q4_K) or tot, plus the bias. Each weight byte is read once per tile of
 * activation rows (the lane-order GEMV of the other entry points reads it
 * once per eight rows). A tolerance claim as the Q8_0 form: within the
 * spec's dequant_matmul_a8 bound (spec/stdlib.md:260-275); each row's result
 * depends on that row alone; refused rows take the reference-order float32
 * path. Returns MIMG_NOT_HANDLED for shapes or weight alignments it does
 * not tile (Q4_K blocks must start 16-byte aligned, Q6_K 2-byte). No
 * reference counterpart: a faster form of the products interp/fast.go:282-379
 * makes, for callers that accept the tolerance. */
int mimg_matmul_a8_quantized_b32_tiled_dev(uint64_t w, const float *x, int64_t rows, const float *bias, float *y,
                                           const void *ws, uint64_t ws_bytes, void *stream);

/* mimg_matmul_a8_quantized_dev for a group of 1 to 3 weights sharing K and
 * the quantized activations (e.g. q, k and v after
 * mimg_rms_norm_quant_dev); bias may be NULL or hold NULLs. No reference
 * counterpart beyond the per-weight fast path it equals bit for bit. */
int mimg_matmul_a8_quantized_group_dev(const uint64_t *w, int count, const float *x, int64_t rows,
                                       const float *const *bias, int block, float *const *y, const void *ws,
                                       uint64_t ws_bytes, void *stream);

/* rms_norm.v1 (reference interp/fast.go:434-485, with the residual add
 * before it) and the 8-bit quantizer of dequant_matmul_a8 (q8.go:50-97) on
 * its output, in one launch: if resid is not NULL, x += resid (written
 * back); y = rms_norm(x) * scale is written and quantized into ws (the
 * layout of mimg_quantize_act_dev for rows, n, block). Equal, bit for bit,
 * to mimg_rms_norm_dev followed by mimg_quantize_act_dev, except that the
 * f64 sum of squares may round differently (~1e-16 relative). x, y, resid,
 * scale 16-byte aligned; n a multiple of block, at most 32768. */
int mimg_rms_norm_quant_dev(float *x, const float *resid, const float *scale, float eps, int64_t rows, int64_t n,
                            float *y, int block, void *ws, uint64_t ws_bytes, void *stream);

/* swiglu.v1 over g, u [rows, n] (as mimg_swiglu_dev over rows*n elements
 * with GOMAXPROCS = procs) and the 8-bit quantizer on its output, in one
 * launch: out is written and quantized into ws. Bit for bit the two calls.
 * 16-byte aligned; n a multiple of block, at most 32768; out must not
 * overlap g or u (MIMG_ERR_ARG): the row's refusal flag is screened from g
 * and u while out is written. */
int mimg_swiglu_quant_dev(const float *g, const float *u, float *out, int64_t rows, int64_t n, int procs, int block,
                          void *ws, uint64_t ws_bytes, void *stream);

/* rope.v1 on q [T, heads, d] (in place) and k [T, kv_heads, d], and the
 * cache scatter of the rotated k and of v into kcache/vcache at
 * cache_index[t], in one launch: bit for bit mimg_rope_dev on q and k then
 * mimg_kv_store_dev (reference importer/llama.go:364-503). k is left as
 * it was. */
int mimg_rope_kv_dev(float *q, const float *k, const float *v, const int64_t *pos, const int64_t *cache_index,
                     const double *inv_freq, int64_t T, int heads, int kv_heads, int d, int rotary, int interleaved,
                     int64_t context, void *kcache, void *vcache, int f16, void *stream);

/* mimg_dequant_matmul on device buffers; y must not overlap x. */
int mimg_linear_f32_dev(uint64_t w, const float *x, int64_t rows, const float *bias, float *y,
                        void *stream);

/* dequant_matmul.v1 for many rows (prefill) on the fp32 matrix cores
 * (reference linearF32/linearCols, interp/fast.go:161-183). Each weight is
 * decoded as mim.Dequantize does, bit for bit; the products are summed in
 * float32 in another order than the reference's, within the bound the spec
 * sets for dequant_matmul.v1 (spec/stdlib.md:230-246):
 * |y - exact| <= (K+1) * 2^-24 * sum_k |x_k w_k|, then bias is added. K must
 * be a multiple of 32 (of 256 for Q4_K and Q6_K); rows <= 65535*128. The
 * rows of W the 8-bit path refuses need no special case here. y must not
 * overlap x. */
int mimg_linear_f32_mfma_dev(uint64_t w, const float *x, int64_t rows, const float *bias, float *y,
                             void *stream);

/* mimg_dequantize on device buffers. */
int mimg_dequantize_dev(uint32_t dtype, const void *src, uint64_t len, float *dst, int64_t n,
                        void *stream);

/* Encodes n float32 values into blocks of dtype on the GPU (dst_len bytes).
 * Q8_0 is the reference's encoder (mim.Quantize, quant.go:165-228). The
 * reference has no Q4_K/Q6_K encoder (quant.go:165-194 returns
 * CodeUnsupportedDType); encoders are not normative (spec/dtypes.md:44-45),
 * and these two are this library's own, for synthetic weights. */
int mimg_quantize_dev(uint32_t dtype, const float *src, int64_t n, void *dst, uint64_t dst_len,
                      void *stream);

/* A plain streaming read of `count` (1..8) device byte ranges (16-byte
 * aligned, lengths non-zero multiples of 16) in one launch: one workgroup of
 * 256 threads per per_thread*4 KB (per_thread 16-byte nontemporal loads
 * each, 2, 4, 8 or 16). sink: 1024 uint32 of device memory, written only
 * for one XOR pattern of the data. No reference counterpart: it measures
 * the read rate a launch of that size reaches on this GPU, the ceiling the
 * HBM-bound products are compared with. */
int mimg_stream_read_dev(const void *const *src, const uint64_t *len, int count, int per_thread, uint32_t *sink,
                         void *stream);

/* n values ~ N(0, stdv^2) into dst (device), a function of (seed, index)
 * only. No reference counterpart: it builds the random weights of the
 * benchmark models (N(0, 0.02^2) before encoding) on the device. */
int mimg_synthetic_normal_dev(uint64_t seed, float stdv, float *dst, int64_t n, void *stream);

/* ---- decoder-step ops on device buffers ---------------------------------
 * The other fast paths of the graph the reference's importer writes for a
 * llama/qwen2 model (reference importer/llama.go:317-547, interp/fast.go:40-59),
 * so that a decoder step's activations stay on the GPU between the linear
 * layers. Float results follow the reference's formulas; they are checked
 * against the reference fixture's float64-oracle logits within its own
 * tolerances, not bit for bit. */

/* embedding.v1 (reference interp/fast.go:818-842): out[t] = the decoded row
 * ids[t] of a registered table [V, E] (Q4_K, Q6_K, Q8_0 or F32); a row of
 * zeros for an id outside 0..V-1, as the reference leaves it. */
int mimg_embedding_dev(uint64_t table, const int32_t *ids, int64_t T, float *out, void *stream);

/* rms_norm.v1 (reference interp/fast.go:434-485), with the graph's residual
 * add before it (importer/llama.go:512-514, 520): if resid is not NULL,
 * x += resid (written back); then y = rms_norm(x) * scale (scale may be NULL).
 * x, y: [rows, n]. */
int mimg_rms_norm_dev(float *x, const float *resid, const float *scale, float eps, int64_t rows, int64_t n, float *y,
                      void *stream);

/* rope.v1 (reference interp/fast.go:507-557, transformer.go:257-324) in place
 * on x [T, heads, d]: angles pos[t] * inv_freq[i] in f64 (inv_freq: device
 * f64 [rotary/2], theta^(-2i/rotary)); adjacent pairs if interleaved. */
int mimg_rope_dev(float *x, const int64_t *pos, const double *inv_freq, int64_t T, int heads, int d, int rotary,
                  int interleaved, void *stream);

/* The cache scatter of the graph (reference importer/llama.go:489-503): k, v
 * [T, kv_heads, d] into the caches at the cache indices pos[t] (slot *
 * per-slot context + position with several slots), rounded to f16 when
 * f16 != 0 (the caches are then f16). Rows whose index is outside
 * 0..context-1 are not stored.
 *
 * Cache layouts (the graph's caches are [kv_heads, context, d]; these hold
 * the same values): kcache is [kv_heads, context, d]; vcache is blocked by
 * eight keys, [kv_heads, ceil(context/8), d, 8]: value (h, j, i) at
 * ((h*ceil(context/8) + j/8)*d + i)*8 + j%8, so that a dim's eight
 * consecutive keys are contiguous for the weighted sum, whose per-dim chain
 * runs over the keys in order. vcache holds kv_heads*ceil(context/8)*8*d
 * elements (mimg_vcache_elems), more than kv_heads*context*d when context
 * is not a multiple of 8: a buffer sized for the graph's layout is too
 * small. */
int mimg_kv_store_dev(const float *k, const float *v, const int64_t *pos, int64_t T, int kv_heads, int d,
                      int64_t context, void *kcache, void *vcache, int f16, void *stream);

/* Elements (f16 or f32, as the cache) of a value cache in the blocked layout
 * above: kv_heads * ceil(context/8) * 8 * d; 0 for a non-positive argument.
 * Every entry point that takes a vcache reads or writes up to this many. */
uint64_t mimg_vcache_elems(int64_t kv_heads, int64_t context, int64_t d);

/* attention.v1 (f32 cache) / attention.v2 (f16 cache) with the graph's
 * mask (reference interp/fast.go:559-700, importer/llama.go:364-395), on
 * caches in the layouts of mimg_kv_store_dev:
 * query t of head h sees the cache entries kstart[t]..kend[t] (inclusive;
 * kstart may be NULL for 0) of kv head h / (heads / kv_heads), as the mask
 * of a cache with one or several sequences ("slots") allows; scale
 * 1/sqrt(d). q, out: [T, heads, d]. Bit for bit the reference's attendRow
 * with its AVX2 kernels (interp/fast.go:728-751; scores, Cephes expf sum
 * and ordered weighted sum of internal/kernels/attn_amd64.s:12-468).
 * d a multiple of 8, at most 512. The visible range is clipped to the
 * cache row and to max_keys (1..8192; the per-sequence context); a query
 * that sees nothing gets zeros, a non-finite largest score NaN. ws: device
 * scratch of mimg_attention_workspace_bytes(T, heads, max_keys) bytes
 * (the scores). */
uint64_t mimg_attention_workspace_bytes(int64_t T, int heads, int64_t max_keys);
int mimg_attention_dev(const float *q, const void *kcache, const void *vcache, const int64_t *kend,
                       const int64_t *kstart, int64_t T, int heads, int kv_heads, int d, int64_t context,
                       int64_t max_keys, int f16, float *out, void *ws, uint64_t ws_bytes, void *stream);

/* One step of the greedy loop on the device (reference cmd/mim-run/main.go
 * generate, 184-257), for n sequences: ids[i] = chosen[i], out[count*n+i] =
 * chosen[i] while count < cap (out holds cap*n ids), pos[i] += 1,
 * cache_index[i] += 1 (if not NULL), count += 1. So a captured decode step
 * needs no host round trip. */
int mimg_greedy_advance_dev(const int32_t *chosen, int32_t *ids, int64_t *pos, int64_t *cache_index, int32_t *out,
                            int32_t *count, int cap, int n, void *stream);

/* swiglu.v1 (reference interp/fast.go:487-498): out = silu(g) * u, bit for
 * bit as the reference computes it with GOMAXPROCS = procs: its parallel()
 * cuts the n elements into pieces of max(1, n / (min(procs, n) * 8))
 * (interp/pool.go:33-51) and SiluMulF32 (internal/kernels/attn.go:63-76)
 * takes the first len&~7 of each piece through the AVX2 formula
 * (attn_amd64.s:459-535), the rest through float64. */
int mimg_swiglu_dev(const float *g, const float *u, float *out, int64_t n, int procs, void *stream);

/* Greedy choice (reference cmd/mim-run/main.go:184-192): out[r] = the first
 * index of the largest value of row r of x [rows, n], as the reference's
 * loop from index 0 with x > v[best]: NaNs are never chosen, and a row
 * whose first value is NaN gives 0. */
int mimg_argmax_dev(const float *x, int64_t rows, int64_t n, int32_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
