// C ABI of libmimg (include/mimg.h): weight registry, per-thread streams and
// buffers, argument checks in the reference's terms, and dispatch to the
// gfx950 kernels. No CPU compute path: every product runs on the GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "../../include/mimg.h"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"

using namespace mimg;

namespace {

thread_local std::string t_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(MIMG_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),     \
                        __FILE__, __LINE__);                                             \
    } while (0)

struct Weight {
    DevWeight dw;
    uint8_t* data = nullptr;
    uint8_t* wref = nullptr;
    uint64_t len = 0;
    bool has_key = false;
    std::tuple<uintptr_t, uint64_t, uint32_t, int64_t, int64_t> key;
    uint64_t fp = 0;    // sampled fingerprint of the host bytes (has_key)
    int64_t refs = 1;   // registrations not yet released
    int64_t inflight = 0;  // calls between their lookup and their return
    bool dead = false;     // released while calls were in flight: the last one frees it
    uint8_t* view_of = nullptr;  // a view into this uploaded weights section (data not owned)
};

// Weights sections uploaded whole (mimg_upload_weights): device base -> (length, live views).
struct Upload {
    uint64_t len;
    int64_t views;
    bool orphan = false;  // mimg_shutdown left it for views still held by calls: the last view frees it
};
std::map<uintptr_t, Upload> g_uploads;

std::mutex g_mu;
int g_device = -1;
// Workgroups of a chain launch: one per CU when the chain kernel fits a CU
// (set by mimg_init), else 0.
int g_chain_wgs = 0;

// Scratch of mimg_linear_a8_noalloc_dev: the quantized activations
// (act_layout) in a file-scope device array, so that the call allocates
// nothing. Each GPU the library runs on holds its own copy until the
// process ends. In host code `scratch` is only a stand-in for the symbol:
// its device address is taken once per device with hipGetSymbolAddress at
// mimg_init and kept in g_scratch; kernels receive that address.
constexpr uint64_t SCRATCH_BYTES = 4ull << 20;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
void* g_scratch[MAX_DEVICES] = {};
uint64_t g_next = 1;
std::unordered_map<uint64_t, Weight*> g_weights;
std::map<std::tuple<uintptr_t, uint64_t, uint32_t, int64_t, int64_t>, uint64_t> g_keys;

// Per-thread stream and grow-only device buffers of the host-memory entry
// points.
struct ThreadCtx {
    hipStream_t stream = nullptr;
    void* buf[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t cap[4] = {0, 0, 0, 0};
    void* pin[3] = {nullptr, nullptr, nullptr};  // pinned host staging: x, bias, y
    size_t pcap[3] = {0, 0, 0};
    void release() {
        for (int i = 0; i < 4; i++) {
            if (buf[i]) (void)hipFree(buf[i]);
            buf[i] = nullptr;
            cap[i] = 0;
        }
        for (int i = 0; i < 3; i++) {
            if (pin[i]) (void)hipHostFree(pin[i]);
            pin[i] = nullptr;
            pcap[i] = 0;
        }
        if (stream) (void)hipStreamDestroy(stream);
        stream = nullptr;
    }
    ~ThreadCtx() { release(); }
};
thread_local ThreadCtx t_ctx;

int64_t block_elems(uint32_t dt) {
    switch (dt) {
    case DT_Q8_0: return 32;
    case DT_Q4_K:
    case DT_Q6_K: return 256;
    }
    return -1;
}
int64_t block_bytes(uint32_t dt) {
    switch (dt) {
    case DT_Q8_0: return Q80_BYTES;
    case DT_Q4_K: return Q4K_BYTES;
    case DT_Q6_K: return Q6K_BYTES;
    }
    return -1;
}

const char* dt_name(uint32_t dt) {
    switch (dt) {
    case DT_Q8_0: return "q8_0";
    case DT_Q4_K: return "q4_k";
    case DT_Q6_K: return "q6_k";
    case DT_F32: return "f32";
    }
    return "?";
}

int ensure_device() {
    if (g_device < 0) return fail(MIMG_ERR_NOT_INIT, "mimg_init has not been called");
    HIP_TRY(hipSetDevice(g_device));
    return MIMG_OK;
}

int ensure_thread_stream() {
    if (!t_ctx.stream) HIP_TRY(hipStreamCreateWithFlags(&t_ctx.stream, hipStreamNonBlocking));
    return MIMG_OK;
}

int thread_buf(int i, size_t bytes, void** out) {
    if (bytes == 0) bytes = 256;
    if (t_ctx.cap[i] < bytes) {
        if (t_ctx.buf[i]) HIP_TRY(hipFree(t_ctx.buf[i]));
        t_ctx.buf[i] = nullptr;
        t_ctx.cap[i] = 0;
        HIP_TRY(hipMalloc(&t_ctx.buf[i], bytes));
        t_ctx.cap[i] = bytes;
    }
    *out = t_ctx.buf[i];
    return MIMG_OK;
}

// Pinned host staging buffer i of the calling thread, grown as needed.
int thread_pin(int i, size_t bytes, void** out) {
    if (bytes == 0) bytes = 256;
    if (t_ctx.pcap[i] < bytes) {
        if (t_ctx.pin[i]) HIP_TRY(hipHostFree(t_ctx.pin[i]));
        t_ctx.pin[i] = nullptr;
        t_ctx.pcap[i] = 0;
        // mapped and coherent: kernels may read and write it in place
        HIP_TRY(hipHostMalloc(&t_ctx.pin[i], bytes, hipHostMallocMapped | hipHostMallocCoherent));
        t_ctx.pcap[i] = bytes;
    }
    *out = t_ctx.pin[i];
    return MIMG_OK;
}

// Frees a weight that is out of the maps and used by no call (g_mu held).
// Kernels enqueued on it by earlier calls may still run: wait for them.
void destroy_locked(Weight* w) {
    (void)hipDeviceSynchronize();
    if (w->view_of) {
        auto it = g_uploads.find((uintptr_t)w->view_of);
        if (it != g_uploads.end() && --it->second.views == 0 && it->second.orphan) {
            (void)hipFree((void*)it->first);
            g_uploads.erase(it);
        }
    } else {
        (void)hipFree(w->data);
    }
    (void)hipFree(w->wref);
    delete w;
}

// Weights released while a call held them: the last holder hands them here
// instead of freeing them itself (a holder may be enqueuing onto a stream
// under graph capture, where synchronising and freeing are not allowed).
// mimg_release_weight, the registrations and mimg_shutdown free them.
std::vector<Weight*> g_grave;
void drain_grave_locked() {
    for (Weight* w : g_grave) destroy_locked(w);
    g_grave.clear();
}

// A weight held by one call from its lookup to its return. While any call
// holds it, mimg_release_weight only unlinks it (no new call can find it)
// and the last holder frees it, so a weight shared by concurrent sessions
// is never freed under a call that is still enqueuing work on it.
class Held {
  public:
    Held() = default;
    Held(const Held&) = delete;
    Held& operator=(const Held&) = delete;
    ~Held() { reset(); }
    int acquire(uint64_t h) {
        reset();
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_weights.find(h);
        if (it == g_weights.end()) return fail(MIMG_ERR_HANDLE, "unknown weight handle %llu", (unsigned long long)h);
        w_ = it->second;
        w_->inflight++;
        return MIMG_OK;
    }
    void reset() {
        if (!w_) return;
        std::lock_guard<std::mutex> lk(g_mu);
        if (--w_->inflight == 0 && w_->dead) g_grave.push_back(w_);
        w_ = nullptr;
    }
    Weight* get() const { return w_; }
    Weight* operator->() const { return w_; }

  private:
    Weight* w_ = nullptr;
};

int check_shape(uint32_t dtype, uint64_t len, int64_t n, int64_t k) {
    int64_t be = block_elems(dtype);
    if (be < 0) return fail(MIMG_NOT_HANDLED, "dtype %u has no kernel", dtype);
    if (n <= 0 || k <= 0) return fail(MIMG_ERR_ARG, "weight shape [%lld, %lld]", (long long)n, (long long)k);
    if (k % be)
        return fail(MIMG_ERR_ARG, "%s: K = %lld is not a multiple of the block size %lld", dt_name(dtype),
                    (long long)k, (long long)be);
    uint64_t want = (uint64_t)n * (uint64_t)(k / be) * (uint64_t)block_bytes(dtype);
    if (len != want)
        return fail(MIMG_ERR_ARG, "%s [%lld, %lld] needs %llu bytes, got %llu", dt_name(dtype), (long long)n,
                    (long long)k, (unsigned long long)want, (unsigned long long)len);
    return MIMG_OK;
}

// A cheap fingerprint of host bytes: 64 evenly spaced 8-byte samples and
// the first and last 64 bytes, mixed with splitmix64's finaliser. It tells
// a registered buffer from other bytes later mapped at the same address (a
// closed and reopened file) without reading the whole tensor on each call.
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static uint64_t fingerprint(const uint8_t* p, uint64_t len) {
    uint64_t h = mix64(len);
    auto take = [&](uint64_t off) {
        uint64_t v = 0;
        const uint64_t m = len - off < 8 ? len - off : 8;
        memcpy(&v, p + off, m);
        h = mix64(h ^ v ^ (off << 1));
    };
    for (uint64_t o = 0; o < 64 && o < len; o += 8) take(o);
    for (uint64_t o = len > 64 ? len - 64 : 0; o < len; o += 8) take(o);
    if (len > 8)
        for (uint64_t i = 0; i < 64; i++) take(i * (len - 8) / 63);
    return h;
}

int register_impl(const void* src, uint64_t len, uint32_t dtype, int64_t n, int64_t k, bool from_host,
                  uint64_t* handle) {
    if (!handle || !src) return fail(MIMG_ERR_ARG, "null pointer");
    int rc = check_shape(dtype, len, n, k);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        drain_grave_locked();
    }
    auto key = std::make_tuple((uintptr_t)src, len, dtype, n, k);
    const uint64_t fp = from_host ? fingerprint((const uint8_t*)src, len) : 0;
    if (from_host) {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_keys.find(key);
        if (it != g_keys.end()) {
            Weight* old = g_weights[it->second];
            if (old->fp == fp) {
                old->refs++;
                *handle = it->second;
                return MIMG_OK;
            }
            // other bytes at a registered address: the old entry keeps its
            // handle until released, the key goes to a fresh upload
            old->has_key = false;
            g_keys.erase(it);
        }
    }
    Weight* w = new Weight();
    hipError_t e = hipMalloc((void**)&w->data, len + WEIGHT_PAD);
    if (e == hipSuccess) e = hipMalloc((void**)&w->wref, (size_t)n);
    if (e == hipSuccess) e = hipMemset(w->data + len, 0, WEIGHT_PAD);
    if (e == hipSuccess)
        e = hipMemcpy(w->data, src, len, from_host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice);
    if (e == hipSuccess) e = launch_weight_refusals(dtype, w->data, n, k, w->wref, nullptr);
    std::vector<uint8_t> flags;
    if (e == hipSuccess) {
        flags.resize((size_t)n);
        e = hipMemcpy(flags.data(), w->wref, (size_t)n, hipMemcpyDeviceToHost);
    }
    if (e != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        if (w->wref) (void)hipFree(w->wref);
        delete w;
        return fail(MIMG_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
    }
    int64_t refused = 0;
    for (uint8_t f : flags) refused += f;
    w->len = len;
    w->dw.dt = dtype;
    w->dw.n = n;
    w->dw.k = k;
    w->dw.row_bytes = k / block_elems(dtype) * block_bytes(dtype);
    w->dw.data = w->data;
    w->dw.wref = w->wref;
    w->dw.n_refused = refused;
    w->has_key = from_host;
    w->key = key;
    w->fp = fp;
    std::lock_guard<std::mutex> lk(g_mu);
    if (from_host) {
        auto it = g_keys.find(key);
        if (it != g_keys.end() && g_weights[it->second]->fp == fp) {  // another thread registered it meanwhile
            (void)hipFree(w->data);
            (void)hipFree(w->wref);
            delete w;
            g_weights[it->second]->refs++;
            *handle = it->second;
            return MIMG_OK;
        }
        if (it != g_keys.end()) g_weights[it->second]->has_key = false;
        g_keys[key] = g_next;
    }
    g_weights[g_next] = w;
    *handle = g_next++;
    return MIMG_OK;
}

bool fused_q8_blocks(uint32_t dt, int block) {
    // FusedQ8Blocks (reference internal/kernels/q8.go:105-117) on a machine
    // with every kernel: blocks of 32 for Q4_K/Q6_K/Q8_0, 256 for Q4_K/Q6_K.
    if (block == 32) return dt == DT_Q4_K || dt == DT_Q6_K || dt == DT_Q8_0;
    if (block == 256) return dt == DT_Q4_K || dt == DT_Q6_K;
    return false;
}

// Activation rows from which the blocks-of-256 products use the MFMA GEMM
// (bit-identical to the GEMV) instead of the GEMV in chunks of eight rows.
constexpr int64_t GEMM_MIN_ROWS = 16;

// Every workgroup of a product reads all of x (the float32 path of refused
// rows included) while others write y: y[i] must not overlap x.
static int check_outputs(const float* x, int64_t rows, int64_t K, const int64_t* N, float* const* y, int count) {
    const uintptr_t xa = (uintptr_t)x, xe = xa + (uint64_t)rows * (uint64_t)K * 4;
    for (int i = 0; i < count; i++) {
        const uintptr_t ya = (uintptr_t)y[i], ye = ya + (uint64_t)rows * (uint64_t)N[i] * 4;
        if (y[i] && ya < xe && xa < ye) return fail(MIMG_ERR_ARG, "output %d overlaps the input x", i);
    }
    return MIMG_OK;
}

// Activation rows (of a chunk of at most eight) from which the GEMV runs
// on the matrix cores (measured, cfg1 layer set: 100 against 105 us per
// step at 4 rows, 99 against 95 at 3).
constexpr int64_t MFMA_MIN_ROWS = 4;

// Everything after quantization: the products of up to three weights (same
// K, each with an 8-bit kernel for `block`) with activations already
// quantized into `a`; block-256 weights of one dtype share a launch per
// chunk of 8 rows. Every path keeps each row's result independent of the
// other rows of the call: block 256 from GEMM_MIN_ROWS on the MFMA GEMM
// (bit-identical to the GEMV), blocks of 32 always the GEMV in the
// reference's lane order.
int matmul_quantized(const Weight* const* w, int count, const float* x, int64_t rows, const float* const* bias,
                     int block, float* const* y, const ActPtrs& a, hipStream_t s) {
    const int64_t K = w[0]->dw.k, R32 = K / 32, R16 = K / 16;
    if (block == 256 && rows >= GEMM_MIN_ROWS) {
        bool all = true;
        for (int i = 0; i < count; i++) all = all && gemm_a8k_ok(w[i]->dw);
        if (all) {
            for (int i = 0; i < count; i++) {
                hipError_t e = launch_gemm_a8k(w[i]->dw, a, rows, rows, x, bias ? bias[i] : nullptr, y[i], s);
                if (e != hipSuccess) return fail(MIMG_ERR_HIP, "GEMM launch: %s", hipGetErrorString(e));
            }
            return MIMG_OK;
        }
    }
    for (int64_t r0 = 0; r0 < rows; r0 += 8) {
        const int64_t mr = rows - r0 < 8 ? rows - r0 : 8;
        ActPtrs c;
        c.q = a.q + r0 * K;
        c.d32 = a.d32 + r0 * R32;
        c.xs = a.xs + r0 * R32;
        c.ys16 = a.ys16 + r0 * R16;
        c.dbs = a.dbs + r0 * R32;
        c.ok = a.ok + r0;
        bool done[3] = {false, false, false};
        for (int i = 0; i < count; i++) {
            if (done[i]) continue;
            hipError_t e;
            if (block == 256) {
                const DevWeight* dws[3];
                const float* bs[3];
                float* ys[3];
                int n = 0;
                for (int j = i; j < count; j++) {
                    if (done[j] || w[j]->dw.dt != w[i]->dw.dt) continue;
                    dws[n] = &w[j]->dw;
                    bs[n] = bias ? bias[j] : nullptr;
                    ys[n] = y[j] + r0 * w[j]->dw.n;
                    done[j] = true;
                    n++;
                }
                if (mr >= MFMA_MIN_ROWS && gemv_mfma_ok(dws, n, mr))
                    e = launch_gemv_a8k_mfma(dws, n, c, mr, rows, x + r0 * K, bs, ys, s);
                else
                    e = launch_gemv_a8k(dws, n, c, mr, rows, x + r0 * K, bs, ys, s);
            } else {
                const int64_t N = w[i]->dw.n;
                if (w[i]->dw.dt == DT_Q8_0)
                    e = launch_gemv_q8_0_a8(w[i]->dw, c, mr, rows, x + r0 * K, bias ? bias[i] : nullptr,
                                            y[i] + r0 * N, N, s);
                else
                    e = launch_gemv_kq_a8_b32(w[i]->dw, c, mr, rows, x + r0 * K, bias ? bias[i] : nullptr,
                                              y[i] + r0 * N, N, s);
                done[i] = true;
            }
            if (e != hipSuccess) return fail(MIMG_ERR_HIP, "product launch: %s", hipGetErrorString(e));
        }
    }
    return MIMG_OK;
}

// Argument checks shared by the 8-bit entry points. Returns > 0 with
// *use_f32 set when the dtype has no 8-bit kernel for `block`.
int a8_checks(const Weight* w, int64_t rows, int block, bool* use_f32) {
    *use_f32 = false;
    if (block != 32 && block != 256)
        return fail(MIMG_ERR_ARG, "dequant_matmul_a8: block must be 32 or 256, got %d", block);
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    if (!fused_q8_blocks(w->dw.dt, block)) {
        *use_f32 = true;
        return MIMG_OK;
    }
    return MIMG_OK;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" {

int mimg_version(void) { return (0 << 16) | 1; }

const char* mimg_last_error(void) { return t_err.c_str(); }

int mimg_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(MIMG_ERR_DEVICE, "device %d of %d", device, count);
    if (g_device >= 0 && g_device != device)
        return fail(MIMG_ERR_DEVICE, "already initialised on device %d", g_device);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MIMG_ERR_DEVICE, "device %d is %s; libmimg is built for gfx950", device, prop.gcnArchName);
    HIP_TRY(hipSetDevice(device));
    if (device >= MAX_DEVICES) return fail(MIMG_ERR_DEVICE, "device %d: at most %d devices", device, MAX_DEVICES);
    if (!g_scratch[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(MIMG_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        g_scratch[device] = p;
    }
    if (chain_occupancy() >= 1) {
        int cus = 0;
        HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
        g_chain_wgs = cus;
    }
    g_device = device;
    return MIMG_OK;
}

void mimg_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_device < 0) return;
    (void)hipSetDevice(g_device);
    (void)hipDeviceSynchronize();
    drain_grave_locked();
    for (auto& kv : g_weights) {
        Weight* w = kv.second;
        if (w->inflight > 0) {
            w->dead = true;  // a call on another thread still holds it: that call hands it to the grave
            continue;
        }
        if (w->view_of) {
            auto it = g_uploads.find((uintptr_t)w->view_of);
            if (it != g_uploads.end()) it->second.views--;
        } else {
            (void)hipFree(w->data);  // a view's bytes belong to its section
        }
        (void)hipFree(w->wref);
        delete w;
    }
    g_weights.clear();
    g_keys.clear();
    for (auto it = g_uploads.begin(); it != g_uploads.end();) {
        if (it->second.views > 0) {  // views still held by calls in flight free it last
            it->second.orphan = true;
            ++it;
        } else {
            (void)hipFree((void*)it->first);
            it = g_uploads.erase(it);
        }
    }
    // the calling thread's stream and buffers; other threads' go at their exit
    t_ctx.release();
    g_device = -1;
}

int mimg_register_weight(const void* host, uint64_t len, uint32_t dtype, int64_t n, int64_t k, uint64_t* handle) {
    return register_impl(host, len, dtype, n, k, true, handle);
}

int mimg_register_weight_device(const void* dev, uint64_t len, uint32_t dtype, int64_t n, int64_t k,
                                uint64_t* handle) {
    return register_impl(dev, len, dtype, n, k, false, handle);
}

int mimg_release_weight(uint64_t handle) {
    int rc = ensure_device();
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_weights.find(handle);
    if (it == g_weights.end()) return fail(MIMG_ERR_HANDLE, "unknown weight handle %llu", (unsigned long long)handle);
    Weight* w = it->second;
    drain_grave_locked();
    if (--w->refs > 0) return MIMG_OK;
    if (w->has_key) g_keys.erase(w->key);
    g_weights.erase(it);
    if (w->inflight > 0) w->dead = true;  // the last call holding it hands it to the grave
    else destroy_locked(w);
    return MIMG_OK;
}

int mimg_upload_weights(const void* host, uint64_t len, void** dev) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!host || !dev || len == 0) return fail(MIMG_ERR_ARG, "null pointer or empty section");
    uint8_t* d = nullptr;
    hipError_t e = hipMalloc((void**)&d, len + WEIGHT_PAD);
    if (e == hipSuccess) e = hipMemset(d + len, 0, WEIGHT_PAD);
    if (e == hipSuccess) e = hipMemcpy(d, host, len, hipMemcpyHostToDevice);  // one transfer
    if (e != hipSuccess) {
        if (d) (void)hipFree(d);
        return fail(MIMG_ERR_HIP, "weights upload (%llu bytes): %s", (unsigned long long)len, hipGetErrorString(e));
    }
    std::lock_guard<std::mutex> lk(g_mu);
    g_uploads[(uintptr_t)d] = Upload{len, 0};
    *dev = d;
    return MIMG_OK;
}

int mimg_free_weights(void* dev) {
    int rc = ensure_device();
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_uploads.find((uintptr_t)dev);
    if (it == g_uploads.end()) return fail(MIMG_ERR_ARG, "not an uploaded weights section");
    if (it->second.views > 0)
        return fail(MIMG_ERR_ARG, "%lld weight views of this section are still registered", (long long)it->second.views);
    g_uploads.erase(it);
    HIP_TRY(hipDeviceSynchronize());
    (void)hipFree(dev);
    return MIMG_OK;
}

int mimg_register_weight_view(const void* dev, uint64_t len, uint32_t dtype, int64_t n, int64_t k, uint64_t* handle) {
    if (!handle || !dev) return fail(MIMG_ERR_ARG, "null pointer");
    int rc = check_shape(dtype, len, n, k);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    uint8_t* base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        drain_grave_locked();
        auto it = g_uploads.upper_bound((uintptr_t)dev);
        if (it != g_uploads.begin()) {
            --it;
            const uintptr_t b = it->first, p = (uintptr_t)dev;
            if (p >= b && p - b <= it->second.len && len <= it->second.len - (p - b)) base = (uint8_t*)b;
        }
        if (!base) return fail(MIMG_ERR_ARG, "the view is not inside an uploaded weights section");
    }
    Weight* w = new Weight();
    hipError_t e = hipMalloc((void**)&w->wref, (size_t)n);
    if (e == hipSuccess) e = launch_weight_refusals(dtype, (const uint8_t*)dev, n, k, w->wref, nullptr);
    std::vector<uint8_t> flags;
    if (e == hipSuccess) {
        flags.resize((size_t)n);
        e = hipMemcpy(flags.data(), w->wref, (size_t)n, hipMemcpyDeviceToHost);
    }
    if (e != hipSuccess) {
        if (w->wref) (void)hipFree(w->wref);
        delete w;
        return fail(MIMG_ERR_HIP, "weight view: %s", hipGetErrorString(e));
    }
    int64_t refused = 0;
    for (uint8_t f : flags) refused += f;
    w->data = (uint8_t*)dev;
    w->view_of = base;
    w->len = len;
    w->dw.dt = dtype;
    w->dw.n = n;
    w->dw.k = k;
    w->dw.row_bytes = k / block_elems(dtype) * block_bytes(dtype);
    w->dw.data = w->data;
    w->dw.wref = w->wref;
    w->dw.n_refused = refused;
    std::lock_guard<std::mutex> lk(g_mu);
    g_uploads[(uintptr_t)base].views++;
    g_weights[g_next] = w;
    *handle = g_next++;
    return MIMG_OK;
}

int mimg_weight_info(uint64_t handle, const void** dev_ptr, int64_t* n_refused) {
    Held w;
    int rc = w.acquire(handle);
    if (rc) return rc;
    if (dev_ptr) *dev_ptr = w->data;
    if (n_refused) *n_refused = w->dw.n_refused;
    return MIMG_OK;
}

uint64_t mimg_a8_workspace_bytes(int64_t rows, int64_t k) {
    if (rows < 0 || k <= 0) return 0;
    return act_layout(rows, k).total;
}

int mimg_a8_workspace_offsets(int64_t rows, int64_t k, uint64_t off[6]) {
    if (rows < 0 || k <= 0 || !off) return fail(MIMG_ERR_ARG, "bad workspace shape");
    ActLayout l = act_layout(rows, k);
    off[0] = l.q;
    off[1] = l.d32;
    off[2] = l.xs;
    off[3] = l.ys16;
    off[4] = l.dbs;
    off[5] = l.ok;
    return MIMG_OK;
}

int mimg_quantize_act_dev(const float* x, int64_t rows, int64_t k, int block, void* ws, uint64_t ws_bytes,
                          void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (block != 32 && block != 256) return fail(MIMG_ERR_ARG, "block must be 32 or 256, got %d", block);
    if (rows < 0 || k <= 0 || k % block) return fail(MIMG_ERR_ARG, "K = %lld with blocks of %d", (long long)k, block);
    if (rows == 0) return MIMG_OK;
    if (!x || !ws || !aligned(x, 16) || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "x must be 16-byte and ws 256-byte aligned");
    ActLayout l = act_layout(rows, k);
    if (ws_bytes < l.total) return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    HIP_TRY(launch_quantize_act(x, rows, k, block, act_ptrs(ws, l), (hipStream_t)stream));
    return MIMG_OK;
}

static int qa_checks(int64_t rows, int64_t k, int block, const void* ws, uint64_t ws_bytes, ActLayout* l) {
    if (block != 32 && block != 256) return fail(MIMG_ERR_ARG, "block must be 32 or 256, got %d", block);
    if (rows < 0 || k <= 0 || k % block) return fail(MIMG_ERR_ARG, "K = %lld with blocks of %d", (long long)k, block);
    if (k > 32768) return fail(MIMG_ERR_ARG, "K = %lld: the fused producers take rows of at most 32768", (long long)k);
    if (rows == 0) return MIMG_OK;
    if (!ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "ws must be 256-byte aligned");
    *l = act_layout(rows, k);
    if (ws_bytes < l->total)
        return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l->total);
    return MIMG_OK;
}

int mimg_rms_norm_quant_dev(float* x, const float* resid, const float* scale, float eps, int64_t rows, int64_t n,
                            float* y, int block, void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    ActLayout l;
    if ((rc = qa_checks(rows, n, block, ws, ws_bytes, &l)) || rows == 0) return rc;
    if (!x || !y || !aligned(x, 16) || !aligned(y, 16) || (resid && !aligned(resid, 16)) || (scale && !aligned(scale, 16)))
        return fail(MIMG_ERR_ARG, "x, y, resid and scale must be 16-byte aligned");
    HIP_TRY(launch_norm_quantize_act(x, resid, scale, eps, y, rows, n, block, act_ptrs(ws, l), (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_swiglu_quant_dev(const float* g, const float* u, float* out, int64_t rows, int64_t n, int procs, int block,
                          void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    ActLayout l;
    if ((rc = qa_checks(rows, n, block, ws, ws_bytes, &l)) || rows == 0) return rc;
    if (!g || !u || !out || !aligned(g, 16) || !aligned(u, 16) || !aligned(out, 16))
        return fail(MIMG_ERR_ARG, "g, u and out must be 16-byte aligned");
    // One workgroup per row screens the whole of g and u for the refusal
    // flag while the others write out: out must be a buffer of its own.
    const uint64_t nbytes = (uint64_t)rows * (uint64_t)n * 4;
    auto overlap = [nbytes](const void* a, const void* b) {
        return (uintptr_t)a < (uintptr_t)b + nbytes && (uintptr_t)b < (uintptr_t)a + nbytes;
    };
    if (overlap(out, g) || overlap(out, u))
        return fail(MIMG_ERR_ARG, "swiglu_quant: out must not overlap g or u");
    const int64_t total = rows * n, w = procs < total ? procs : total;
    int64_t chunk = total;
    if (w > 1) chunk = total / (w * 8) > 1 ? total / (w * 8) : 1;
    HIP_TRY(launch_swiglu_quantize_act(g, u, out, chunk, rows, n, block, act_ptrs(ws, l), (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_rope_kv_dev(float* q, const float* k, const float* v, const int64_t* pos, const int64_t* cache_index,
                     const double* inv_freq, int64_t T, int heads, int kv_heads, int d, int rotary, int interleaved,
                     int64_t context, void* kcache, void* vcache, int f16, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (T < 0 || T > 65535 || heads <= 0 || kv_heads <= 0 || d <= 0 || d % 2 || d > 1024 || rotary <= 0 ||
        rotary % 2 || rotary > d || context <= 0)
        return fail(MIMG_ERR_ARG, "rope_kv: T %lld, heads %d, kv heads %d, D %d, rotary %d", (long long)T, heads, kv_heads,
                    d, rotary);
    if (T == 0) return MIMG_OK;
    if (!q || !k || !v || !pos || !cache_index || !inv_freq || !kcache || !vcache)
        return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_rope_kv(q, k, v, pos, cache_index, inv_freq, (int)T, heads, kv_heads, d, rotary, interleaved, context,
                           kcache, vcache, f16, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_matmul_a8_quantized_group_dev(const uint64_t* whs, int count, const float* x, int64_t rows,
                                       const float* const* bias, int block, float* const* y, const void* ws,
                                       uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !y || count < 1 || count > 3) return fail(MIMG_ERR_ARG, "a group holds 1 to 3 weights, got %d", count);
    Held held[3];
    const Weight* w[3];
    for (int i = 0; i < count; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        Weight* wi = held[i].get();
        bool use_f32;
        if ((rc = a8_checks(wi, rows, block, &use_f32))) return rc;
        if (use_f32) return fail(MIMG_ERR_ARG, "%s has no 8-bit kernel for blocks of %d", dt_name(wi->dw.dt), block);
        if (wi->dw.k != (i ? w[0]->dw.k : wi->dw.k)) return fail(MIMG_ERR_ARG, "the weights of a group must share K");
        w[i] = wi;
    }
    if (rows == 0) return MIMG_OK;
    if (!x || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    ActLayout l = act_layout(rows, w[0]->dw.k);
    if (ws_bytes < l.total)
        return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    const float* bs[3];
    float* ys[3];
    int64_t ns[3];
    for (int i = 0; i < count; i++) {
        bs[i] = bias ? bias[i] : nullptr;
        ys[i] = y[i];
        ns[i] = w[i]->dw.n;
    }
    if ((rc = check_outputs(x, rows, w[0]->dw.k, ns, ys, count))) return rc;
    return matmul_quantized(w, count, x, rows, bs, block, ys, act_ptrs((void*)ws, l), (hipStream_t)stream);
}

int mimg_linear_f32_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, float* y, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    if (rows == 0) return MIMG_OK;
    if (!x || !y) return fail(MIMG_ERR_ARG, "null pointer");
    if ((rc = check_outputs(x, rows, w->dw.k, &w->dw.n, &y, 1))) return rc;
    HIP_TRY(launch_linear_f32(w->dw, x, rows, bias, y, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_linear_f32_mfma_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, float* y, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    if (rows < 0 || rows > INT32_MAX) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    if (rows == 0) return MIMG_OK;
    if (!x || !y) return fail(MIMG_ERR_ARG, "null pointer");
    if ((rc = check_outputs(x, rows, w->dw.k, &w->dw.n, &y, 1))) return rc;
    if ((rows + 127) / 128 > 65535) return fail(MIMG_ERR_ARG, "rows = %lld: more than 65535 tiles of 128", (long long)rows);
    HIP_TRY(launch_linear_f32_mfma(w->dw, x, rows, bias, y, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_matmul_a8_quantized_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, int block, float* y,
                                 const void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    bool use_f32;
    if ((rc = a8_checks(w.get(), rows, block, &use_f32))) return rc;
    if (use_f32) return fail(MIMG_ERR_ARG, "%s has no 8-bit kernel for blocks of %d", dt_name(w->dw.dt), block);
    if (rows == 0) return MIMG_OK;
    if (!x || !y || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    ActLayout l = act_layout(rows, w->dw.k);
    if (ws_bytes < l.total) return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    if ((rc = check_outputs(x, rows, w->dw.k, &w->dw.n, &y, 1))) return rc;
    const Weight* ws1[1] = {w.get()};
    const float* bs1[1] = {bias};
    float* ys1[1] = {y};
    return matmul_quantized(ws1, 1, x, rows, bs1, block, ys1, act_ptrs((void*)ws, l), (hipStream_t)stream);
}

int mimg_matmul_a8_quantized_q8_0_tiled_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, float* y,
                                            const void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    if (w->dw.dt != DT_Q8_0) return fail(MIMG_ERR_ARG, "%s: the tiled product is for Q8_0 weights", dt_name(w->dw.dt));
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    if (rows == 0) return MIMG_OK;
    if (!x || !y || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    ActLayout l = act_layout(rows, w->dw.k);
    if (ws_bytes < l.total) return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    if ((rc = check_outputs(x, rows, w->dw.k, &w->dw.n, &y, 1))) return rc;
    if (!gemm_q8_0_ok(w->dw)) return fail(MIMG_NOT_HANDLED, "no tiled Q8_0 product for this shape");
    HIP_TRY(launch_gemm_q8_0(w->dw, act_ptrs((void*)ws, l), rows, rows, x, bias, y, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_matmul_a8_quantized_b32_tiled_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, float* y,
                                           const void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    const uint32_t dt = w->dw.dt;
    if (dt != DT_Q8_0 && dt != DT_Q4_K && dt != DT_Q6_K)
        return fail(MIMG_ERR_ARG, "%s: the tiled products with blocks of 32 are for Q8_0, Q4_K and Q6_K weights",
                    dt_name(dt));
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    if (rows == 0) return MIMG_OK;
    if (!x || !y || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    ActLayout l = act_layout(rows, w->dw.k);
    if (ws_bytes < l.total) return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    if ((rc = check_outputs(x, rows, w->dw.k, &w->dw.n, &y, 1))) return rc;
    if (dt == DT_Q8_0) {
        if (!gemm_q8_0_ok(w->dw)) return fail(MIMG_NOT_HANDLED, "no tiled Q8_0 product for this shape");
        HIP_TRY(launch_gemm_q8_0(w->dw, act_ptrs((void*)ws, l), rows, rows, x, bias, y, (hipStream_t)stream));
        return MIMG_OK;
    }
    // the tile copies take Q4_K blocks as whole 16-byte chunks and Q6_K
    // blocks from the 16-byte boundary below them (even addresses)
    if (!gemm_kq_b32_ok(w->dw) || !aligned(w->dw.data, dt == DT_Q4_K ? 16 : 2))
        return fail(MIMG_NOT_HANDLED, "no tiled %s product with blocks of 32 for this shape or alignment", dt_name(dt));
    HIP_TRY(launch_gemm_kq_b32(w->dw, act_ptrs((void*)ws, l), rows, rows, x, bias, y, (hipStream_t)stream));
    return MIMG_OK;
}

// When a single activation row is quantized inside the GEMV kernel: every
// workgroup then quantizes the whole row, which pays while the group is
// small (q/k/v, o); for long rows or many weight rows a separate quantize
// launch costs less (measured on MI355X).
constexpr int64_t FUSED_MAX_K = 4096, FUSED_MAX_N = 8192;

int mimg_linear_a8_group_dev(const uint64_t* whs, int count, const float* x, int64_t rows, const float* const* bias,
                             int block, float* const* y, void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !y || count < 1 || count > 3) return fail(MIMG_ERR_ARG, "a group holds 1 to 3 weights, got %d", count);
    Held held[3];
    Weight* w[3];
    const DevWeight* dw[3];
    bool all_f32 = true, any_f32 = false;
    for (int i = 0; i < count; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        w[i] = held[i].get();
        if (w[i]->dw.k != w[0]->dw.k) return fail(MIMG_ERR_ARG, "the weights of a group must share K");
        bool use_f32;
        if ((rc = a8_checks(w[i], rows, block, &use_f32))) return rc;
        all_f32 = all_f32 && use_f32;
        any_f32 = any_f32 || use_f32;
        dw[i] = &w[i]->dw;
    }
    if (rows == 0) return MIMG_OK;
    if (!x || !aligned(x, 16)) return fail(MIMG_ERR_ARG, "x must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    int64_t total_n = 0, ns[3];
    for (int i = 0; i < count; i++) total_n += (ns[i] = w[i]->dw.n);
    if ((rc = check_outputs(x, rows, w[0]->dw.k, ns, y, count))) return rc;
    if (!any_f32 && rows == 1 && block == 256 && w[0]->dw.k <= FUSED_MAX_K && total_n <= FUSED_MAX_N &&
        fused_gemv_ok(dw, count)) {
        float* ys[3];
        const float* bs[3];
        for (int i = 0; i < count; i++) {
            ys[i] = y[i];
            bs[i] = bias ? bias[i] : nullptr;
        }
        HIP_TRY(launch_gemv_a8k_fused(dw, count, x, bs, ys, s));
        return MIMG_OK;
    }
    // The weights without an 8-bit kernel for `block` take the float32 path;
    // the others share one quantization of x.
    const Weight* wa[3];
    const float* ba[3];
    float* ya[3];
    int na = 0;
    for (int i = 0; i < count; i++) {
        const float* bi = bias ? bias[i] : nullptr;
        bool use_f32;
        a8_checks(w[i], rows, block, &use_f32);
        if (use_f32) {
            if ((rc = mimg_linear_f32_dev(whs[i], x, rows, bi, y[i], stream))) return rc;
            continue;
        }
        wa[na] = w[i];
        ba[na] = bi;
        ya[na] = y[i];
        na++;
    }
    (void)all_f32;
    if (na == 0) return MIMG_OK;
    if ((rc = mimg_quantize_act_dev(x, rows, w[0]->dw.k, block, ws, ws_bytes, stream))) return rc;
    ActLayout l = act_layout(rows, w[0]->dw.k);
    return matmul_quantized(wa, na, x, rows, ba, block, ya, act_ptrs(ws, l), s);
}

int mimg_linear_a8_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, int block, float* y, void* ws,
                       uint64_t ws_bytes, void* stream) {
    const float* bs[1] = {bias};
    float* ys[1] = {y};
    return mimg_linear_a8_group_dev(&wh, 1, x, rows, bs, block, ys, ws, ws_bytes, stream);
}

// The most rows any of G workgroups gets of a chain phase: the kernel's
// byte-balanced split (workgroup g takes the rows starting in bytes
// [floor(g*B/G), floor((g+1)*B/G)) of the phase's B weight bytes).
static int64_t chain_max_wg_rows(const ChainPhase& P, int G) {
    auto row_at = [&](int64_t b) {
        int64_t start = 0, base = 0;
        for (int i = 0; i < P.nmat; i++) {
            const int64_t rb = P.m[i].rb, end = start + (int64_t)P.m[i].N * rb;
            if (b <= end || i == P.nmat - 1) {
                const int64_t num = b > start ? b - start : 0;
                int64_t q = (num + rb - 1) / rb;
                if (q > P.m[i].N) q = P.m[i].N;
                return base + q;
            }
            start = end;
            base += P.m[i].N;
        }
        return base;
    };
    int64_t most = 0, prev = row_at(0);
    for (int g = 0; g < G; g++) {
        const int64_t next = row_at(P.bytes * (g + 1) / G);
        if (next - prev > most) most = next - prev;
        prev = next;
    }
    return most;
}

uint64_t mimg_chain_sync_bytes(void) { return CHAIN_SYNC_BYTES; }

uint64_t mimg_vcache_elems(int64_t kv_heads, int64_t context, int64_t d) {
    if (kv_heads <= 0 || context <= 0 || d <= 0) return 0;
    return (uint64_t)kv_heads * (uint64_t)((context + 7) / 8 * 8) * (uint64_t)d;
}

int mimg_chain_sync_init(void* sync, uint64_t sync_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!sync || !aligned(sync, 256) || sync_bytes < CHAIN_SYNC_BYTES)
        return fail(MIMG_ERR_ARG, "sync must be 256-byte aligned and hold mimg_chain_sync_bytes() = %llu bytes",
                    (unsigned long long)CHAIN_SYNC_BYTES);
    HIP_TRY(launch_chain_zero(sync, CHAIN_SYNC_BYTES, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_chain_status(void* sync, uint32_t* status) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!sync || !status) return fail(MIMG_ERR_ARG, "sync and status must not be null");
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(status, sync, 4, hipMemcpyDeviceToHost));
    const uint32_t zero = 0;
    HIP_TRY(hipMemcpy(sync, &zero, 4, hipMemcpyHostToDevice));
    return MIMG_OK;
}

int mimg_linear_a8_chain_dev(const mimg_chain_phase* phases, int nphase, void* sync, uint64_t sync_bytes,
                             void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!phases || nphase < 1 || nphase > CHAIN_MAXP)
        return fail(MIMG_ERR_ARG, "a chain holds 1 to %d phases, got %d", CHAIN_MAXP, nphase);
    if (!sync || !aligned(sync, 256) || sync_bytes < CHAIN_SYNC_BYTES)
        return fail(MIMG_ERR_ARG, "sync must be 256-byte aligned and hold mimg_chain_sync_bytes() = %llu bytes",
                    (unsigned long long)CHAIN_SYNC_BYTES);
    const int cus = g_chain_wgs;
    if (cus <= 0) return fail(MIMG_NOT_HANDLED, "the chain kernel cannot be resident on this device");
    Held held[CHAIN_MAXP * 3];
    ChainArgs A;
    memset(&A, 0, sizeof A);
    for (int p = 0; p < nphase; p++) {
        const mimg_chain_phase& ph = phases[p];
        if (ph.count < 1 || ph.count > 3) return fail(MIMG_ERR_ARG, "phase %d: a group holds 1 to 3 weights, got %d", p, ph.count);
        if (!ph.x || !aligned(ph.x, 16)) return fail(MIMG_ERR_ARG, "phase %d: x must be 16-byte aligned", p);
        ChainPhase& P = A.ph[p];
        P.x = ph.x;
        P.nmat = ph.count;
        int64_t ns[3];
        for (int i = 0; i < ph.count; i++) {
            Held& h = held[3 * p + i];
            if ((rc = h.acquire(ph.w[i]))) return rc;
            const DevWeight& dw = h->dw;
            if (i > 0 && dw.k != P.K) return fail(MIMG_ERR_ARG, "phase %d: the weights of a group must share K", p);
            if (!ph.y[i]) return fail(MIMG_ERR_ARG, "phase %d: output %d is null", p, i);
            if (dw.dt != DT_Q4_K && dw.dt != DT_Q6_K)
                return fail(MIMG_NOT_HANDLED, "phase %d: %s has no chain kernel", p, dt_name(dw.dt));
            if (dw.k % 256 || dw.k > CHAIN_MAXK || dw.row_bytes % 16 || dw.row_bytes > CHAIN_STAGE_BYTES ||
                dw.n > (1 << 30))
                return fail(MIMG_NOT_HANDLED, "phase %d: %s [%lld, %lld] does not fit the chain's stages", p,
                            dt_name(dw.dt), (long long)dw.n, (long long)dw.k);
            P.K = (int32_t)dw.k;
            P.nb = (int32_t)(dw.k / 256);
            ChainMat& M = P.m[i];
            M.W = dw.data;
            M.wref = dw.wref;
            M.bias = ph.bias[i];
            M.y = ph.y[i];
            M.N = (int32_t)dw.n;
            M.dt = (int32_t)dw.dt;
            M.rb = (int32_t)dw.row_bytes;
            M.nref = dw.n_refused > 0 ? 1 : 0;
            const int64_t by_bytes = CHAIN_STAGE_BYTES / dw.row_bytes, by_pairs = CHAIN_MAX_PAIRS / P.nb;
            M.rps = (int32_t)(by_bytes < by_pairs ? by_bytes : by_pairs);
            P.bytes += dw.n * dw.row_bytes;
            ns[i] = dw.n;
        }
        if ((rc = check_outputs(ph.x, 1, P.K, ns, ph.y, ph.count))) return rc;
        if (chain_max_wg_rows(P, cus) * P.nb > CHAIN_TABLE_ENTRIES)
            return fail(MIMG_NOT_HANDLED, "phase %d: more than %d (row, block) pairs for a workgroup", p,
                        CHAIN_TABLE_ENTRIES);
        for (int i = 0; i < ph.count; i++)
            for (int j = i + 1; j < ph.count; j++) {
                const uintptr_t a0 = (uintptr_t)ph.y[i], a1 = a0 + (uint64_t)ns[i] * 4;
                const uintptr_t b0 = (uintptr_t)ph.y[j], b1 = b0 + (uint64_t)ns[j] * 4;
                if (a0 < b1 && b0 < a1) return fail(MIMG_ERR_ARG, "phase %d: outputs %d and %d overlap", p, i, j);
            }
    }
    A.nphase = nphase;
    A.G = cus;
    A.lines = cus < CHAIN_LINES ? cus : CHAIN_LINES;
    A.sync = (uint64_t*)sync;
    HIP_TRY(launch_chain(A, (hipStream_t)stream));
    return MIMG_OK;
}

// Independent one-row groups (each a mimg_linear_a8_group_dev call with one
// activation row and blocks of 256): one launch quantizes every group's row,
// one launch runs every product. Checks shared by the entry point and the
// workspace query; fills held[] and the per-group K.
static int set_checks(const mimg_chain_phase* groups, int ngroups, Held* held, int64_t* K) {
    if (!groups || ngroups < 1 || ngroups > MIMG_SET_MAX_GROUPS)
        return fail(MIMG_ERR_ARG, "a set holds 1 to %d groups, got %d", MIMG_SET_MAX_GROUPS, ngroups);
    int nmat = 0;
    for (int g = 0; g < ngroups; g++) {
        const mimg_chain_phase& gr = groups[g];
        if (gr.count < 1 || gr.count > 3) return fail(MIMG_ERR_ARG, "group %d: a group holds 1 to 3 weights, got %d", g, gr.count);
        if (nmat + gr.count > SET_MAXSEG) return fail(MIMG_ERR_ARG, "a set holds at most %d weights", SET_MAXSEG);
        for (int i = 0; i < gr.count; i++) {
            int rc;
            Held& h = held[nmat++];
            if ((rc = h.acquire(gr.w[i]))) return rc;
            const DevWeight& dw = h->dw;
            if (i == 0) K[g] = dw.k;
            else if (dw.k != K[g]) return fail(MIMG_ERR_ARG, "group %d: the weights of a group must share K", g);
            if (dw.dt != DT_Q4_K && dw.dt != DT_Q6_K)
                return fail(MIMG_NOT_HANDLED, "group %d: %s has no set kernel", g, dt_name(dw.dt));
            if (dw.k % 256 || dw.k > 65536 || dw.n > (1 << 30) || dw.n * dw.row_bytes > ((int64_t)1 << 32))
                return fail(MIMG_NOT_HANDLED, "group %d: %s [%lld, %lld] does not fit the set kernel", g,
                            dt_name(dw.dt), (long long)dw.n, (long long)dw.k);
        }
    }
    return MIMG_OK;
}

int mimg_linear_a8_set_workspace_bytes(const mimg_chain_phase* groups, int ngroups, uint64_t* bytes) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!bytes) return fail(MIMG_ERR_ARG, "bytes is null");
    Held held[MIMG_SET_MAX_GROUPS * 3];
    int64_t K[MIMG_SET_MAX_GROUPS];
    if ((rc = set_checks(groups, ngroups, held, K))) return rc;
    uint64_t total = 0;
    for (int g = 0; g < ngroups; g++) total += act_layout(1, K[g]).total;
    *bytes = total;
    return MIMG_OK;
}

// quantize: the set call (x -> ws, then the products); otherwise the
// products of rows already quantized into ws in the same layout.
static int set_impl(const mimg_chain_phase* groups, int ngroups, void* ws, uint64_t ws_bytes, void* stream,
                    bool quantize) {
    int rc = ensure_device();
    if (rc) return rc;
    Held held[MIMG_SET_MAX_GROUPS * 3];
    int64_t K[MIMG_SET_MAX_GROUPS];
    if ((rc = set_checks(groups, ngroups, held, K))) return rc;
    uint64_t need = 0;
    for (int g = 0; g < ngroups; g++) need += act_layout(1, K[g]).total;
    if (!ws || !aligned(ws, 256) || ws_bytes < need)
        return fail(MIMG_ERR_WORKSPACE, "the set needs a 256-byte aligned workspace of %llu bytes (got %llu)",
                    (unsigned long long)need, (unsigned long long)ws_bytes);
    // Every output against every input and every other output: the
    // quantizer reads each x, and refused rows read x inside the product
    // launch while the other workgroups write their outputs.
    struct Span {
        uintptr_t a, e;
    };
    Span xs[MIMG_SET_MAX_GROUPS], ys[MIMG_SET_MAX_GROUPS * 3];
    int ny = 0, m = 0;
    QaSetArgs Q;
    memset(&Q, 0, sizeof Q);
    SetArgs S;
    memset(&S, 0, sizeof S);
    int qwgs = 0;
    uint64_t off = 0;
    for (int g = 0; g < ngroups; g++) {
        const mimg_chain_phase& gr = groups[g];
        if (!gr.x || !aligned(gr.x, 16)) return fail(MIMG_ERR_ARG, "group %d: x must be 16-byte aligned", g);
        xs[g] = {(uintptr_t)gr.x, (uintptr_t)gr.x + (uint64_t)K[g] * 4};
        const ActLayout l = act_layout(1, K[g]);
        const ActPtrs a = act_ptrs((uint8_t*)ws + off, l);
        off += l.total;
        QaSetRow& qr = Q.row[g];
        qr.x = gr.x;
        qr.K = K[g];
        qr.a = a;
        qr.wg0 = qwgs;
        qwgs += 1 + (int)((K[g] / 256 + 7) / 8);
        for (int i = 0; i < gr.count; i++, m++) {
            const DevWeight& dw = held[m]->dw;
            if (!gr.y[i]) return fail(MIMG_ERR_ARG, "group %d: output %d is null", g, i);
            ys[ny++] = {(uintptr_t)gr.y[i], (uintptr_t)gr.y[i] + (uint64_t)dw.n * 4};
            SetSeg& s = S.seg[m];
            s.W = dw.data;
            s.wref = dw.wref;
            s.bias = gr.bias[i];
            s.y = gr.y[i];
            s.q = a.q;
            s.d32 = a.d32;
            s.s16 = dw.dt == DT_Q4_K ? a.xs : a.ys16;
            s.ok = a.ok;
            s.x = gr.x;
            s.rb = dw.row_bytes;
            s.K = dw.k;
            s.N = (int32_t)dw.n;
            s.nb = (int32_t)(dw.k / 256);
            s.dt = (int32_t)dw.dt;
        }
    }
    for (int i = 0; i < ny; i++) {
        for (int g = 0; g < ngroups; g++)
            if (ys[i].a < xs[g].e && xs[g].a < ys[i].e) return fail(MIMG_ERR_ARG, "output %d overlaps the input of group %d", i, g);
        for (int j = i + 1; j < ny; j++)
            if (ys[i].a < ys[j].e && ys[j].a < ys[i].e) return fail(MIMG_ERR_ARG, "outputs %d and %d overlap", i, j);
    }
    Q.nrows = ngroups;
    S.nseg = m;
    hipStream_t s = (hipStream_t)stream;
    if (quantize) HIP_TRY(launch_quantize_act_set(Q, qwgs, s));
    HIP_TRY(launch_gemv_a8k_set(S, s));
    return MIMG_OK;
}

int mimg_linear_a8_set_dev(const mimg_chain_phase* groups, int ngroups, void* ws, uint64_t ws_bytes, void* stream) {
    return set_impl(groups, ngroups, ws, ws_bytes, stream, true);
}

int mimg_matmul_a8_quantized_set_dev(const mimg_chain_phase* groups, int ngroups, void* ws, uint64_t ws_bytes,
                                     void* stream) {
    return set_impl(groups, ngroups, ws, ws_bytes, stream, false);
}

int mimg_linear_a8_noalloc_dev(uint64_t wh, const float* x, int64_t rows, const float* bias, int block, float* y,
                               void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    void* ws = g_scratch[g_device];
    if (!ws) return fail(MIMG_ERR_NOT_INIT, "no scratch address for device %d", g_device);
    int64_t K;
    {
        Held w;
        if ((rc = w.acquire(wh))) return rc;
        K = w->dw.k;
    }
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    // (rows past SCRATCH_BYTES / K cannot fit; checked before the size
    // arithmetic, which a huge rows value would overflow)
    const uint64_t need = (uint64_t)rows > SCRATCH_BYTES / (uint64_t)K ? SCRATCH_BYTES + 1 : act_layout(rows, K).total;
    if (need > SCRATCH_BYTES)
        return fail(MIMG_ERR_WORKSPACE,
                    "%lld rows x K = %lld need %llu bytes of scratch; the library's static scratch holds %llu "
                    "(call mimg_linear_a8_dev with a workspace instead)",
                    (long long)rows, (long long)K, (unsigned long long)need, (unsigned long long)SCRATCH_BYTES);
    return mimg_linear_a8_dev(wh, x, rows, bias, block, y, ws, SCRATCH_BYTES, stream);
}

uint64_t mimg_noalloc_scratch_bytes(void) { return SCRATCH_BYTES; }

int mimg_rms_norm_linear_a8_group_dev(const uint64_t* whs, int count, const float* x, const float* resid,
                                      const float* scale, float eps, float* x_out, const float* const* bias,
                                      float* const* y, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !y || count < 1 || count > 3) return fail(MIMG_ERR_ARG, "a group holds 1 to 3 weights, got %d", count);
    if (!x || !x_out || !aligned(x, 16) || !aligned(x_out, 16) || (resid && !aligned(resid, 16)) ||
        (scale && !aligned(scale, 16)))
        return fail(MIMG_ERR_ARG, "x, x_out, resid and scale must be non-null (resid, scale may be null) and 16-byte aligned");
    Held held[3];
    Weight* w[3];
    const DevWeight* dw[3];
    int64_t total_n = 0;
    for (int i = 0; i < count; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        w[i] = held[i].get();
        if (w[i]->dw.k != w[0]->dw.k) return fail(MIMG_ERR_ARG, "the weights of a group must share K");
        bool use_f32;
        if ((rc = a8_checks(w[i], 1, 256, &use_f32))) return rc;
        if (use_f32) return fail(MIMG_NOT_HANDLED, "%s has no 8-bit kernel for blocks of 256", dt_name(w[i]->dw.dt));
        dw[i] = &w[i]->dw;
        total_n += w[i]->dw.n;
    }
    const int64_t K = w[0]->dw.k;
    const uint64_t xb = (uint64_t)K * 4;
    auto overlap = [xb](const void* a, const void* b) {
        return b && (uintptr_t)a < (uintptr_t)b + xb && (uintptr_t)b < (uintptr_t)a + xb;
    };
    if (overlap(x_out, x) || overlap(x_out, resid) || overlap(x_out, scale))
        return fail(MIMG_ERR_ARG, "x_out must not overlap x, resid or scale (every workgroup reads them)");
    // Every workgroup reads x, resid and scale and writes its share of x_out
    // and y: an output y[i] must overlap none of those four buffers.
    for (int i = 0; i < count; i++) {
        const uintptr_t ya = (uintptr_t)y[i], ye = ya + (uint64_t)w[i]->dw.n * 4;
        auto hits = [&](const void* b) {
            return b && ya < (uintptr_t)b + xb && (uintptr_t)b < ye;
        };
        if (!y[i]) return fail(MIMG_ERR_ARG, "output %d is null", i);
        if (hits(x) || hits(resid) || hits(scale) || hits(x_out))
            return fail(MIMG_ERR_ARG, "output %d overlaps x, resid, scale or x_out", i);
    }
    if (total_n > FUSED_MAX_N || !fused_norm_ok(dw, count))
        return fail(MIMG_NOT_HANDLED, "no fused norm GEMV for K %lld, %lld rows", (long long)K, (long long)total_n);
    float* ys[3];
    const float* bs[3];
    for (int i = 0; i < count; i++) {
        ys[i] = y[i];
        bs[i] = bias ? bias[i] : nullptr;
    }
    HIP_TRY(launch_gemv_a8k_fused_norm(dw, count, x, resid, scale, eps, x_out, bs, ys, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_matmul_a8_quantized_swiglu_dev(const uint64_t* whs, const float* x, int64_t rows, const float* const* bias,
                                        int block, float* out, int procs, const void* ws, uint64_t ws_bytes,
                                        void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !out) return fail(MIMG_ERR_ARG, "null pointer");
    Held held[2];
    const Weight* w[2];
    for (int i = 0; i < 2; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        Weight* wi = held[i].get();
        bool use_f32;
        if ((rc = a8_checks(wi, rows, block, &use_f32))) return rc;
        if (use_f32) return fail(MIMG_ERR_ARG, "%s has no 8-bit kernel for blocks of %d", dt_name(wi->dw.dt), block);
        w[i] = wi;
    }
    if (rows == 0) return MIMG_OK;
    // one row: the pair kernel's epilogue; 2..8 rows: the matrix-core GEMV's
    const bool one = rows == 1 && gemv_swiglu_ok(w[0]->dw, w[1]->dw);
    const bool few = rows >= 2 && rows <= 8 && gemv_mfma_swiglu_ok(w[0]->dw, w[1]->dw, rows);
    if (block != 256 || !(one || few))
        return fail(MIMG_NOT_HANDLED, "no swiglu epilogue for %lld rows, block %d, %s/%s", (long long)rows, block,
                    dt_name(w[0]->dw.dt), dt_name(w[1]->dw.dt));
    if (!x || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    const int64_t K = w[0]->dw.k, N = w[0]->dw.n;
    ActLayout l = act_layout(rows, K);
    if (ws_bytes < l.total)
        return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    int64_t ns[1] = {N};
    float* ys[1] = {out};
    if ((rc = check_outputs(x, rows, K, ns, ys, 1))) return rc;
    if ((uintptr_t)out < (uintptr_t)ws + ws_bytes && (uintptr_t)ws < (uintptr_t)out + (uint64_t)(rows * N) * 4)
        return fail(MIMG_ERR_ARG, "out overlaps the workspace");
    // swiglu.v1's pieces over the flattened [rows, N] products (the
    // reference's parallel(): GOMAXPROCS procs)
    const int64_t total = rows * N, wk = procs < total ? procs : total;
    int64_t chunk = total;
    if (wk > 1) chunk = total / (wk * 8) > 1 ? total / (wk * 8) : 1;
    const float* bs[2] = {bias ? bias[0] : nullptr, bias ? bias[1] : nullptr};
    if (one)
        HIP_TRY(launch_gemv_a8k_swiglu(w[0]->dw, w[1]->dw, act_ptrs((void*)ws, l), x, bs, out, total, chunk,
                                       (hipStream_t)stream));
    else
        HIP_TRY(launch_gemv_a8k_mfma_swiglu(w[0]->dw, w[1]->dw, act_ptrs((void*)ws, l), rows, x, bs, out, total,
                                            chunk, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_matmul_a8_quantized_qkv_rope_kv_dev(const uint64_t* whs, const float* x, int64_t rows,
                                             const float* const* bias, int block, float* q, const int64_t* pos,
                                             const int64_t* cache_index, const double* inv_freq, int heads,
                                             int kv_heads, int d, int rotary, int interleaved, int64_t context,
                                             void* kcache, void* vcache, int f16, const void* ws, uint64_t ws_bytes,
                                             void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !q || !pos || !cache_index || !inv_freq || !kcache || !vcache) return fail(MIMG_ERR_ARG, "null pointer");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || d <= 0 || d % 2 || d > 1024 || rotary <= 0 || rotary % 2 ||
        rotary > d || context <= 0)
        return fail(MIMG_ERR_ARG, "rope: heads %d, kv heads %d, D %d, rotary %d, context %lld", heads, kv_heads, d,
                    rotary, (long long)context);
    Held held[3];
    const DevWeight* dw[3];
    for (int i = 0; i < 3; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        Weight* w = held[i].get();
        if (w->dw.k != held[0].get()->dw.k) return fail(MIMG_ERR_ARG, "q, k and v must share K");
        bool use_f32;
        if ((rc = a8_checks(w, rows, block, &use_f32))) return rc;
        if (use_f32) return fail(MIMG_NOT_HANDLED, "%s has no 8-bit kernel for blocks of %d", dt_name(w->dw.dt), block);
        dw[i] = &w->dw;
    }
    if (rows == 0) return MIMG_OK;
    if (block != 256 || rows < MFMA_MIN_ROWS || rows > 8 || dw[0]->dt != dw[1]->dt ||
        !gemv_mfma_qkv_ok(dw, rows, heads, kv_heads, d, rotary))
        return fail(MIMG_NOT_HANDLED, "no q/k/v + rope launch for %lld rows, block %d, D %d", (long long)rows, block, d);
    if (!x || !ws || !aligned(ws, 256)) return fail(MIMG_ERR_ARG, "null or misaligned pointer");
    const int64_t K = dw[0]->k;
    ActLayout l = act_layout(rows, K);
    if (ws_bytes < l.total)
        return fail(MIMG_ERR_WORKSPACE, "workspace %llu < %llu bytes", (unsigned long long)ws_bytes, (unsigned long long)l.total);
    int64_t ns[1] = {dw[0]->n};
    float* ys[1] = {q};
    if ((rc = check_outputs(x, rows, K, ns, ys, 1))) return rc;
    const float* bs[3] = {bias ? bias[0] : nullptr, bias ? bias[1] : nullptr, bias ? bias[2] : nullptr};
    HIP_TRY(launch_gemv_a8k_mfma_qkv(dw, act_ptrs((void*)ws, l), rows, x, bs, q, pos, cache_index, inv_freq, heads,
                                     kv_heads, d, rotary, interleaved, context, kcache, vcache, f16,
                                     (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_rms_norm_qkv_rope_kv_dev(const uint64_t* whs, const float* x, const float* resid, const float* scale,
                                  float eps, float* x_out, const float* const* bias, float* q, const int64_t* pos,
                                  const int64_t* cache_index, const double* inv_freq, int heads, int kv_heads, int d,
                                  int rotary, int interleaved, int64_t context, void* kcache, void* vcache, int f16,
                                  void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!whs || !x || !x_out || !q || !pos || !cache_index || !inv_freq || !kcache || !vcache)
        return fail(MIMG_ERR_ARG, "null pointer");
    if (!aligned(x, 16) || !aligned(x_out, 16) || (resid && !aligned(resid, 16)) || (scale && !aligned(scale, 16)))
        return fail(MIMG_ERR_ARG, "x, x_out, resid and scale must be 16-byte aligned");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || d <= 0 || d % 2 || d > 1024 || rotary <= 0 || rotary % 2 ||
        rotary > d || context <= 0)
        return fail(MIMG_ERR_ARG, "rope: heads %d, kv heads %d, D %d, rotary %d, context %lld", heads, kv_heads, d,
                    rotary, (long long)context);
    Held held[3];
    const DevWeight* dw[3];
    for (int i = 0; i < 3; i++) {
        if ((rc = held[i].acquire(whs[i]))) return rc;
        Weight* w = held[i].get();
        if (w->dw.k != held[0].get()->dw.k) return fail(MIMG_ERR_ARG, "q, k and v must share K");
        bool use_f32;
        if ((rc = a8_checks(w, 1, 256, &use_f32))) return rc;
        if (use_f32) return fail(MIMG_NOT_HANDLED, "%s has no 8-bit kernel for blocks of 256", dt_name(w->dw.dt));
        dw[i] = &w->dw;
    }
    const int64_t K = dw[0]->k;
    const uint64_t xb = (uint64_t)K * 4, qb = (uint64_t)dw[0]->n * 4;
    auto overlap = [](const void* a, uint64_t la, const void* b, uint64_t lb) {
        return a && b && (uintptr_t)a < (uintptr_t)b + lb && (uintptr_t)b < (uintptr_t)a + la;
    };
    if (overlap(x_out, xb, x, xb) || overlap(x_out, xb, resid, xb) || overlap(x_out, xb, scale, xb))
        return fail(MIMG_ERR_ARG, "x_out must not overlap x, resid or scale (every workgroup reads them)");
    if (overlap(q, qb, x, xb) || overlap(q, qb, resid, xb) || overlap(q, qb, scale, xb) || overlap(q, qb, x_out, xb))
        return fail(MIMG_ERR_ARG, "q overlaps x, resid, scale or x_out");
    if ((int64_t)heads * d + 2 * (int64_t)kv_heads * d > FUSED_MAX_N ||
        !fused_norm_rope_ok(dw, heads, kv_heads, d, rotary))
        return fail(MIMG_NOT_HANDLED, "no fused norm + q/k/v + rope launch for K %lld, D %d", (long long)K, d);
    const float* bs[3] = {bias ? bias[0] : nullptr, bias ? bias[1] : nullptr, bias ? bias[2] : nullptr};
    FusedRope r;
    r.pos = pos;
    r.cidx = cache_index;
    r.inv_freq = inv_freq;
    r.heads = heads;
    r.kv_heads = kv_heads;
    r.d = d;
    r.rotary = rotary;
    r.interleaved = interleaved;
    r.f16 = f16;
    r.context = context;
    r.kcache = kcache;
    r.vcache = vcache;
    HIP_TRY(launch_gemv_a8k_fused_norm_rope(dw, x, resid, scale, eps, x_out, bs, q, r, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_dequantize_dev(uint32_t dtype, const void* src, uint64_t len, float* dst, int64_t n, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    int64_t be = block_elems(dtype);
    if (be < 0) return fail(MIMG_NOT_HANDLED, "cannot decode dtype %u on the GPU", dtype);
    if (n < 0 || n % be) return fail(MIMG_ERR_ARG, "%s: %lld elements is not a multiple of the block size %lld", dt_name(dtype), (long long)n, (long long)be);
    if ((uint64_t)(n / be * block_bytes(dtype)) != len)
        return fail(MIMG_ERR_ARG, "%s: %lld elements need %lld bytes, got %llu", dt_name(dtype), (long long)n,
                    (long long)(n / be * block_bytes(dtype)), (unsigned long long)len);
    if (n == 0) return MIMG_OK;
    HIP_TRY(launch_dequantize(dtype, (const uint8_t*)src, n, dst, (hipStream_t)stream));
    return MIMG_OK;
}

// ---- decoder-step ops ------------------------------------------------------

int mimg_embedding_dev(uint64_t table, const int32_t* ids, int64_t T, float* out, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(table))) return rc;
    if (T < 0 || T > (1 << 30)) return fail(MIMG_ERR_ARG, "T = %lld", (long long)T);
    if (T == 0) return MIMG_OK;
    if (!ids || !out) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_embed_rows(w->dw.dt, w->dw.data, w->dw.row_bytes, ids, (int)T, (int)w->dw.n, w->dw.k, out,
                              (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_rms_norm_dev(float* x, const float* resid, const float* scale, float eps, int64_t rows, int64_t n, float* y,
                      void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (rows < 0 || n <= 0 || rows > (1 << 30)) return fail(MIMG_ERR_ARG, "rows %lld, n %lld", (long long)rows, (long long)n);
    if (rows == 0) return MIMG_OK;
    if (!x || !y) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_rms_norm(x, resid, scale, eps, rows, n, y, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_rope_dev(float* x, const int64_t* pos, const double* inv_freq, int64_t T, int heads, int d, int rotary,
                  int interleaved, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (T < 0 || heads <= 0 || d <= 0 || rotary <= 0 || rotary % 2 || rotary > d)
        return fail(MIMG_ERR_ARG, "rope: T %lld, heads %d, D %d, rotary %d", (long long)T, heads, d, rotary);
    if (T == 0) return MIMG_OK;
    if (!x || !pos || !inv_freq) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_rope(x, pos, inv_freq, (int)T, heads, d, rotary, interleaved, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_kv_store_dev(const float* k, const float* v, const int64_t* pos, int64_t T, int kv_heads, int d,
                      int64_t context, void* kcache, void* vcache, int f16, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (T < 0 || kv_heads <= 0 || d <= 0 || context <= 0) return fail(MIMG_ERR_ARG, "kv store shape");
    if (T == 0) return MIMG_OK;
    if (!k || !v || !pos || !kcache || !vcache) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_kv_store(k, v, pos, (int)T, kv_heads, d, context, kcache, vcache, f16, (hipStream_t)stream));
    return MIMG_OK;
}

uint64_t mimg_attention_workspace_bytes(int64_t T, int heads, int64_t max_keys) {
    if (T < 0 || heads <= 0 || max_keys <= 0) return 0;
    return ((uint64_t)T * (uint64_t)heads * (uint64_t)max_keys * 4 + 255) & ~(uint64_t)255;
}

int mimg_attention_dev(const float* q, const void* kcache, const void* vcache, const int64_t* kend,
                       const int64_t* kstart, int64_t T, int heads, int kv_heads, int d, int64_t context,
                       int64_t max_keys, int f16, float* out, void* ws, uint64_t ws_bytes, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (T < 0 || T > 65535 || heads <= 0 || heads > 65535 || kv_heads <= 0 || heads % kv_heads || d <= 0 || d > 512 ||
        d % 8 || context <= 0)
        return fail(MIMG_ERR_ARG, "attention: T %lld, heads %d, kv heads %d, D %d, context %lld (D a multiple of 8, <= 512)",
                    (long long)T, heads, kv_heads, d, (long long)context);
    if (max_keys < 1 || max_keys > 8192)
        return fail(MIMG_ERR_ARG, "attention: max_keys %lld (1..8192)", (long long)max_keys);
    if (T == 0) return MIMG_OK;
    if (!q || !kcache || !vcache || !kend || !out || !ws) return fail(MIMG_ERR_ARG, "null pointer");
    if (ws_bytes < mimg_attention_workspace_bytes(T, heads, max_keys))
        return fail(MIMG_ERR_WORKSPACE, "attention workspace %llu < %llu bytes", (unsigned long long)ws_bytes,
                    (unsigned long long)mimg_attention_workspace_bytes(T, heads, max_keys));
    HIP_TRY(launch_attention(q, kcache, vcache, kend, kstart, (int)T, heads, kv_heads, d, context, max_keys, f16, out,
                             (float*)ws, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_greedy_advance_dev(const int32_t* chosen, int32_t* ids, int64_t* pos, int64_t* cache_index, int32_t* out,
                            int32_t* count, int cap, int n, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (n < 1 || n > 1024 || cap < 0) return fail(MIMG_ERR_ARG, "greedy advance: %d sequences (1..1024), cap %d", n, cap);
    if (!chosen || !ids || !pos || !out || !count) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_greedy_advance(chosen, ids, pos, cache_index, out, count, cap, n, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_swiglu_dev(const float* g, const float* u, float* out, int64_t n, int procs, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (n < 0) return fail(MIMG_ERR_ARG, "n = %lld", (long long)n);
    if (n == 0) return MIMG_OK;
    if (!g || !u || !out) return fail(MIMG_ERR_ARG, "null pointer");
    // the reference's piece size (interp/pool.go:33-39)
    const int64_t w = procs < n ? procs : n;
    int64_t chunk = n;
    if (w > 1) chunk = n / (w * 8) > 1 ? n / (w * 8) : 1;
    HIP_TRY(launch_swiglu(g, u, out, n, chunk, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_argmax_dev(const float* x, int64_t rows, int64_t n, int32_t* out, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (rows < 0 || n <= 0 || n >= (1ll << 31)) return fail(MIMG_ERR_ARG, "argmax: rows %lld, n %lld", (long long)rows, (long long)n);
    if (rows == 0) return MIMG_OK;
    if (!x || !out) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_argmax(x, rows, n, out, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_synthetic_normal_dev(uint64_t seed, float stdv, float* dst, int64_t n, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (n < 0) return fail(MIMG_ERR_ARG, "n = %lld", (long long)n);
    if (n == 0) return MIMG_OK;
    if (!dst) return fail(MIMG_ERR_ARG, "null pointer");
    HIP_TRY(launch_normal_fill(seed, stdv, dst, n, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_quantize_dev(uint32_t dtype, const float* src, int64_t n, void* dst, uint64_t dst_len, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    int64_t be = block_elems(dtype);
    if (be < 0) return fail(MIMG_NOT_HANDLED, "cannot encode dtype %u", dtype);
    if (n < 0 || n % be) return fail(MIMG_ERR_ARG, "%s: %lld elements is not a multiple of the block size %lld", dt_name(dtype), (long long)n, (long long)be);
    if ((uint64_t)(n / be * block_bytes(dtype)) != dst_len)
        return fail(MIMG_ERR_ARG, "%s: %lld elements need %lld bytes, got %llu", dt_name(dtype), (long long)n,
                    (long long)(n / be * block_bytes(dtype)), (unsigned long long)dst_len);
    if (n == 0) return MIMG_OK;
    HIP_TRY(launch_encode(dtype, src, n, (uint8_t*)dst, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_stream_read_dev(const void* const* src, const uint64_t* len, int count, int per_thread, uint32_t* sink,
                         void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!src || !len || !sink || count < 1 || count > READ_MAX_RANGES)
        return fail(MIMG_ERR_ARG, "stream read: 1 to %d ranges and a sink", READ_MAX_RANGES);
    if (per_thread != 2 && per_thread != 4 && per_thread != 8 && per_thread != 16)
        return fail(MIMG_ERR_ARG, "stream read: %d loads per thread (2, 4, 8 or 16)", per_thread);
    ReadRanges r{};
    r.count = count;
    for (int i = 0; i < count; i++) {
        if (!src[i] || len[i] == 0 || len[i] % 16 || !aligned(src[i], 16))
            return fail(MIMG_ERR_ARG, "stream read: range %d must be 16-byte aligned, a non-zero multiple of 16", i);
        r.src[i] = (const uint8_t*)src[i];
        r.len[i] = (int64_t)len[i];
    }
    HIP_TRY(launch_stream_read(r, per_thread, sink, (hipStream_t)stream));
    return MIMG_OK;
}

int mimg_dequantize(uint32_t dtype, const void* src, uint64_t len, float* dst, int64_t n) {
    int rc = ensure_device();
    if (rc) return rc;
    int64_t be = block_elems(dtype);
    if (be < 0) return fail(MIMG_NOT_HANDLED, "cannot decode dtype %u on the GPU", dtype);
    if (n < 0 || n % be || (uint64_t)(n / be * block_bytes(dtype)) != len)
        return fail(MIMG_ERR_ARG, "%s: %lld elements and %llu bytes do not match", dt_name(dtype), (long long)n, (unsigned long long)len);
    if (n == 0) return MIMG_OK;
    if ((rc = ensure_thread_stream())) return rc;
    void *s_d, *d_d;
    if ((rc = thread_buf(0, len + WEIGHT_PAD, &s_d))) return rc;
    if ((rc = thread_buf(1, (size_t)n * 4, &d_d))) return rc;
    hipStream_t s = t_ctx.stream;
    HIP_TRY(hipMemcpyAsync(s_d, src, len, hipMemcpyHostToDevice, s));
    HIP_TRY(launch_dequantize(dtype, (const uint8_t*)s_d, n, (float*)d_d, s));
    HIP_TRY(hipMemcpyAsync(dst, d_d, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return MIMG_OK;
}

// Host calls whose x and y together take at most this many bytes run on
// the pinned buffers in place.
constexpr size_t HOST_DIRECT_BYTES = 1 << 20;

static int host_call(uint64_t wh, const float* x, int64_t rows, const float* bias, int block, float* y, bool a8) {
    int rc = ensure_device();
    if (rc) return rc;
    Held w;
    if ((rc = w.acquire(wh))) return rc;
    if (rows < 0) return fail(MIMG_ERR_ARG, "rows = %lld", (long long)rows);
    bool use_f32 = !a8;
    if (a8 && (rc = a8_checks(w.get(), rows, block, &use_f32))) return rc;
    if (rows == 0) return MIMG_OK;
    if (!x || !y) return fail(MIMG_ERR_ARG, "null pointer");
    if ((rc = ensure_thread_stream())) return rc;
    const int64_t K = w->dw.k, N = w->dw.n;
    const size_t xb = (size_t)(rows * K * 4), yb = (size_t)(rows * N * 4), bb = (size_t)N * 4;
    void *x_d, *y_d, *b_d = nullptr, *ws = nullptr, *x_p, *y_p, *b_p = nullptr;
    uint64_t wsb = act_layout(rows, K).total;
    if (!use_f32 && (rc = thread_buf(3, wsb, &ws))) return rc;
    // The caller's x, bias and y are pageable (a Go slice): they pass through
    // the thread's pinned buffers, and the call synchronises once.
    if ((rc = thread_pin(0, xb, &x_p))) return rc;
    if ((rc = thread_pin(2, yb, &y_p))) return rc;
    if (bias && (rc = thread_pin(1, bb, &b_p))) return rc;
    memcpy(x_p, x, xb);
    if (bias) memcpy(b_p, bias, bb);
    hipStream_t s = t_ctx.stream;
    if (!use_f32 && xb + yb <= HOST_DIRECT_BYTES) {
        // Small 8-bit calls (decode rows): the quantizer reads x once and
        // the products write y in the pinned buffers themselves, so the call
        // is two kernels and one synchronisation, with no copy commands.
        // (Only rows taking the float32 path read x again. The fused
        // producers and the float32 kernels read x in every workgroup: they
        // take copies.)
        void *xm, *ym, *bm = nullptr;
        HIP_TRY(hipHostGetDevicePointer(&xm, x_p, 0));
        HIP_TRY(hipHostGetDevicePointer(&ym, y_p, 0));
        if (bias) HIP_TRY(hipHostGetDevicePointer(&bm, b_p, 0));
        const float* bs[1] = {(const float*)bm};
        float* ys[1] = {(float*)ym};
        if ((rc = mimg_quantize_act_dev((const float*)xm, rows, K, block, ws, wsb, s))) return rc;
        if ((rc = mimg_matmul_a8_quantized_group_dev(&wh, 1, (const float*)xm, rows, bs, block, ys, ws, wsb, s)))
            return rc;
        HIP_TRY(hipStreamSynchronize(s));
        memcpy(y, y_p, yb);
        return MIMG_OK;
    }
    if ((rc = thread_buf(0, xb, &x_d))) return rc;
    if ((rc = thread_buf(1, yb, &y_d))) return rc;
    if (bias && (rc = thread_buf(2, bb, &b_d))) return rc;
    HIP_TRY(hipMemcpyAsync(x_d, x_p, xb, hipMemcpyHostToDevice, s));
    if (bias) HIP_TRY(hipMemcpyAsync(b_d, b_p, bb, hipMemcpyHostToDevice, s));
    if (use_f32)
        rc = mimg_linear_f32_dev(wh, (const float*)x_d, rows, (const float*)b_d, (float*)y_d, s);
    else
        rc = mimg_linear_a8_dev(wh, (const float*)x_d, rows, (const float*)b_d, block, (float*)y_d, ws, wsb, s);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(y_p, y_d, yb, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    memcpy(y, y_p, yb);
    return MIMG_OK;
}

int mimg_dequant_matmul_a8(uint64_t w, const float* x, int64_t rows, const float* bias, int block, float* y) {
    return host_call(w, x, rows, bias, block, y, true);
}

int mimg_dequant_matmul(uint64_t w, const float* x, int64_t rows, const float* bias, float* y) {
    return host_call(w, x, rows, bias, 0, y, false);
}

}  // extern "C"

namespace mimg {

static size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

ActLayout act_layout(int64_t rows, int64_t K) {
    ActLayout l;
    size_t r = (size_t)rows, k = (size_t)K;
    l.q = 0;
    l.d32 = up256(l.q + r * k);
    l.xs = up256(l.d32 + r * (k / 32) * 4);
    l.ys16 = up256(l.xs + r * (k / 32) * 2);
    l.dbs = up256(l.ys16 + r * (k / 16) * 2);
    l.ok = up256(l.dbs + r * (k / 32) * 4);
    l.total = up256(l.ok + r * 4);
    return l;
}

ActPtrs act_ptrs(void* base, const ActLayout& l) {
    uint8_t* b = (uint8_t*)base;
    ActPtrs a;
    a.q = (int8_t*)(b + l.q);
    a.d32 = (float*)(b + l.d32);
    a.xs = (int16_t*)(b + l.xs);
    a.ys16 = (int16_t*)(b + l.ys16);
    a.dbs = (float*)(b + l.dbs);
    a.ok = (int32_t*)(b + l.ok);
    return a;
}

}  // namespace mimg
