"""Python view of libmimg's C ABI (include/mimg.h).

The reference's host side is Go: interp's fast paths (interp/fast.go:40-59)
call the quantized products through `fastFunc`. Go is not in this image, so
the Go cgo shim (go/mimg_fast.go) is shipped as source and this module plays
its role for tests and benchmarks: the same calls, argument meaning and
error behaviour (status > 0 = not handled, < 0 = error).

Every product runs in libmimg.so on the GPU; there is no CPU fallback. If the
library is missing or the device is not gfx950, calls raise.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# MIMG_LIB selects another build of the library (e.g. one made with other
# compile-time tile parameters).
LIB_PATH = os.environ.get("MIMG_LIB") or os.path.join(HERE, "libmimg.so")

F32, Q8_0, Q4_K, Q6_K = 1, 64, 66, 67
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210}

OK, NOT_HANDLED = 0, 1

# Every exported symbol of include/mimg.h with (restype, argtypes).
_P, _I64, _I, _U32, _U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64
SIGNATURES = {
    "mimg_init": (_I, [_I]),
    "mimg_shutdown": (None, []),
    "mimg_last_error": (ctypes.c_char_p, []),
    "mimg_version": (_I, []),
    "mimg_register_weight": (_I, [_P, _U64, _U32, _I64, _I64, ctypes.POINTER(_U64)]),
    "mimg_register_weight_device": (_I, [_P, _U64, _U32, _I64, _I64, ctypes.POINTER(_U64)]),
    "mimg_release_weight": (_I, [_U64]),
    "mimg_weight_info": (_I, [_U64, ctypes.POINTER(_P), ctypes.POINTER(_I64)]),
    "mimg_dequant_matmul_a8": (_I, [_U64, _P, _I64, _P, _I, _P]),
    "mimg_dequant_matmul": (_I, [_U64, _P, _I64, _P, _P]),
    "mimg_dequantize": (_I, [_U32, _P, _U64, _P, _I64]),
    "mimg_a8_workspace_bytes": (_U64, [_I64, _I64]),
    "mimg_a8_workspace_offsets": (_I, [_I64, _I64, ctypes.POINTER(_U64)]),
    "mimg_quantize_act_dev": (_I, [_P, _I64, _I64, _I, _P, _U64, _P]),
    "mimg_linear_a8_dev": (_I, [_U64, _P, _I64, _P, _I, _P, _P, _U64, _P]),
    "mimg_linear_a8_group_dev": (_I, [ctypes.POINTER(_U64), _I, _P, _I64, ctypes.POINTER(_P), _I,
                                      ctypes.POINTER(_P), _P, _U64, _P]),
    "mimg_linear_a8_chain_dev": (_I, [_P, _I, _P, _U64, _P]),
    "mimg_linear_a8_set_dev": (_I, [_P, _I, _P, _U64, _P]),
    "mimg_linear_a8_set_workspace_bytes": (_I, [_P, _I, ctypes.POINTER(_U64)]),
    "mimg_matmul_a8_quantized_set_dev": (_I, [_P, _I, _P, _U64, _P]),
    "mimg_chain_sync_bytes": (_U64, []),
    "mimg_vcache_elems": (_U64, [_I64, _I64, _I64]),
    "mimg_chain_sync_init": (_I, [_P, _U64, _P]),
    "mimg_chain_status": (_I, [_P, ctypes.POINTER(_U32)]),
    "mimg_rms_norm_linear_a8_group_dev": (_I, [ctypes.POINTER(_U64), _I, _P, _P, _P, ctypes.c_float, _P,
                                               ctypes.POINTER(_P), ctypes.POINTER(_P), _P]),
    "mimg_matmul_a8_quantized_swiglu_dev": (_I, [ctypes.POINTER(_U64), _P, _I64, ctypes.POINTER(_P), _I, _P, _I, _P,
                                                 _U64, _P]),
    "mimg_matmul_a8_quantized_qkv_rope_kv_dev": (_I, [ctypes.POINTER(_U64), _P, _I64, ctypes.POINTER(_P), _I, _P, _P,
                                                      _P, _P, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _P, _U64, _P]),
    "mimg_rms_norm_qkv_rope_kv_dev": (_I, [ctypes.POINTER(_U64), _P, _P, _P, ctypes.c_float, _P, ctypes.POINTER(_P),
                                           _P, _P, _P, _P, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _P]),
    "mimg_matmul_a8_quantized_dev": (_I, [_U64, _P, _I64, _P, _I, _P, _P, _U64, _P]),
    "mimg_matmul_a8_quantized_q8_0_tiled_dev": (_I, [_U64, _P, _I64, _P, _P, _P, _U64, _P]),
    "mimg_matmul_a8_quantized_b32_tiled_dev": (_I, [_U64, _P, _I64, _P, _P, _P, _U64, _P]),
    "mimg_linear_f32_dev": (_I, [_U64, _P, _I64, _P, _P, _P]),
    "mimg_linear_f32_mfma_dev": (_I, [_U64, _P, _I64, _P, _P, _P]),
    "mimg_dequantize_dev": (_I, [_U32, _P, _U64, _P, _I64, _P]),
    "mimg_quantize_dev": (_I, [_U32, _P, _I64, _P, _U64, _P]),
    "mimg_synthetic_normal_dev": (_I, [_U64, ctypes.c_float, _P, _I64, _P]),
    "mimg_upload_weights": (_I, [_P, _U64, ctypes.POINTER(_P)]),
    "mimg_free_weights": (_I, [_P]),
    "mimg_register_weight_view": (_I, [_P, _U64, _U32, _I64, _I64, ctypes.POINTER(_U64)]),
    "mimg_matmul_a8_quantized_group_dev": (_I, [ctypes.POINTER(_U64), _I, _P, _I64, ctypes.POINTER(_P), _I,
                                                ctypes.POINTER(_P), _P, _U64, _P]),
    "mimg_rms_norm_quant_dev": (_I, [_P, _P, _P, ctypes.c_float, _I64, _I64, _P, _I, _P, _U64, _P]),
    "mimg_swiglu_quant_dev": (_I, [_P, _P, _P, _I64, _I64, _I, _I, _P, _U64, _P]),
    "mimg_rope_kv_dev": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _P]),
    "mimg_embedding_dev": (_I, [_U64, _P, _I64, _P, _P]),
    "mimg_rms_norm_dev": (_I, [_P, _P, _P, ctypes.c_float, _I64, _I64, _P, _P]),
    "mimg_rope_dev": (_I, [_P, _P, _P, _I64, _I, _I, _I, _I, _P]),
    "mimg_kv_store_dev": (_I, [_P, _P, _P, _I64, _I, _I, _I64, _P, _P, _I, _P]),
    "mimg_attention_workspace_bytes": (_U64, [_I64, _I, _I64]),
    "mimg_attention_dev": (_I, [_P, _P, _P, _P, _P, _I64, _I, _I, _I, _I64, _I64, _I, _P, _P, _U64, _P]),
    "mimg_greedy_advance_dev": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "mimg_swiglu_dev": (_I, [_P, _P, _P, _I64, _I, _P]),
    "mimg_argmax_dev": (_I, [_P, _I64, _I64, _P, _P]),
    "mimg_stream_read_dev": (_I, [ctypes.POINTER(_P), ctypes.POINTER(_U64), _I, _I, _P, _P]),
    "mimg_linear_a8_noalloc_dev": (_I, [_U64, _P, _I64, _P, _I, _P, _P]),
    "mimg_noalloc_scratch_bytes": (_U64, []),
}


class MimgError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libmimg error {code}: {msg}")
        self.code = code


class NotHandled(MimgError):
    pass


_lib = None


def load(path=LIB_PATH):
    """Loads libmimg.so (no GPU call)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `make -C mimir-model_amd` (or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != OK:
        msg = load().mimg_last_error().decode(errors="replace")
        if rc > 0:
            raise NotHandled(rc, msg)
        raise MimgError(rc, msg)


_inited = False


def init(device=0):
    global _inited
    if not _inited:
        _check(load().mimg_init(device))
        _inited = True


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


class Weight:
    """A weight matrix uploaded once, byte for byte, in its block layout."""

    def __init__(self, data, dt, n, k, device=False, view=False):
        init()
        self.dt, self.n, self.k = dt, n, k
        h = _U64()
        if view:
            # data: (device address inside an uploaded weights section, nbytes)
            ptr, nbytes = data
            _check(load().mimg_register_weight_view(ctypes.c_void_p(ptr), nbytes, dt, n, k, ctypes.byref(h)))
            self._host = None
        elif device:
            # data: (device pointer, nbytes)
            ptr, nbytes = data
            _check(load().mimg_register_weight_device(ctypes.c_void_p(ptr), nbytes, dt, n, k, ctypes.byref(h)))
            self._host = None
        else:
            self._host = np.ascontiguousarray(data, dtype=np.uint8)
            _check(load().mimg_register_weight(_p(self._host), self._host.size, dt, n, k, ctypes.byref(h)))
        self.handle = h.value

    def info(self):
        p, nref = _P(), _I64()
        _check(load().mimg_weight_info(self.handle, ctypes.byref(p), ctypes.byref(nref)))
        return p.value, nref.value

    def release(self):
        if self.handle:
            _check(load().mimg_release_weight(self.handle))
            self.handle = 0

    def __del__(self):
        # each Weight holds one reference of its registration
        try:
            self.release()
        except Exception:
            pass


class WeightsSection:
    """A container's weights section uploaded whole (mimg_upload_weights)."""

    def __init__(self, host):
        init()
        host = np.ascontiguousarray(np.frombuffer(host, np.uint8) if not isinstance(host, np.ndarray) else host)
        p = _P()
        _check(load().mimg_upload_weights(_p(host), host.size, ctypes.byref(p)))
        self.ptr, self.nbytes = p.value, host.size

    def view(self, offset, nbytes, dt, n, k):
        if offset < 0 or offset + nbytes > self.nbytes:
            raise ValueError(f"view [{offset}, +{nbytes}) outside the section of {self.nbytes} bytes")
        return Weight((self.ptr + offset, nbytes), dt, n, k, view=True)

    def free(self):
        if self.ptr:
            _check(load().mimg_free_weights(_P(self.ptr)))
            self.ptr = 0


def dequant_matmul_a8(w, x, bias=None, block=256):
    """dequant_matmul_a8.v1/v2 on host arrays: x [..., K] f32 -> y [..., N]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.size // w.k
    y = np.empty(x.shape[:-1] + (w.n,), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(load().mimg_dequant_matmul_a8(w.handle, _p(x), rows, _p(b), block, _p(y)))
    return y


def dequant_matmul(w, x, bias=None):
    """dequant_matmul.v1 on host arrays."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.size // w.k
    y = np.empty(x.shape[:-1] + (w.n,), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(load().mimg_dequant_matmul(w.handle, _p(x), rows, _p(b), _p(y)))
    return y


def dequantize(dt, raw, n):
    init()
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8) if not isinstance(raw, np.ndarray) else raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    _check(load().mimg_dequantize(dt, _p(raw), raw.size, _p(out), n))
    return out


def a8_workspace_bytes(rows, k):
    return int(load().mimg_a8_workspace_bytes(rows, k))


def a8_workspace_offsets(rows, k):
    off = (_U64 * 6)()
    _check(load().mimg_a8_workspace_offsets(rows, k, off))
    return [int(v) for v in off]


# ---- device-pointer calls (pointers and streams as Python ints) ----------

def quantize_act_dev(x_ptr, rows, k, block, ws_ptr, ws_bytes, stream):
    _check(load().mimg_quantize_act_dev(_P(x_ptr), rows, k, block, _P(ws_ptr), ws_bytes, _P(stream)))


def linear_a8_dev(w, x_ptr, rows, bias_ptr, block, y_ptr, ws_ptr, ws_bytes, stream):
    _check(load().mimg_linear_a8_dev(w.handle, _P(x_ptr), rows, _P(bias_ptr) if bias_ptr else None, block,
                                     _P(y_ptr), _P(ws_ptr), ws_bytes, _P(stream)))


def linear_a8_noalloc_dev(w, x_ptr, rows, bias_ptr, block, y_ptr, stream):
    """mimg_linear_a8_dev with the library's static scratch (no workspace,
    no allocation)."""
    _check(load().mimg_linear_a8_noalloc_dev(w.handle, _P(x_ptr), rows, _P(bias_ptr) if bias_ptr else None, block,
                                             _P(y_ptr), _P(stream)))


def linear_a8_group_dev(weights, x_ptr, rows, bias_ptrs, block, y_ptrs, ws_ptr, ws_bytes, stream):
    """Weights sharing one input (e.g. q, k, v): y_ptrs[i] = x . W_i^T (+ bias)."""
    n = len(weights)
    hs = (_U64 * n)(*[w.handle for w in weights])
    ys = (_P * n)(*[_P(p) for p in y_ptrs])
    bs = None if bias_ptrs is None else (_P * n)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_linear_a8_group_dev(hs, n, _P(x_ptr), rows, bs, block, ys,
                                           _P(ws_ptr) if ws_ptr else None, ws_bytes, _P(stream)))


class _ChainPhase(ctypes.Structure):
    """mimg_chain_phase (include/mimg.h)."""
    _fields_ = [("x", _P), ("count", _I), ("w", _U64 * 3), ("bias", _P * 3), ("y", _P * 3)]


def chain_sync_bytes():
    return int(load().mimg_chain_sync_bytes())


def chain_sync_init(sync_ptr, sync_bytes, stream):
    _check(load().mimg_chain_sync_init(_P(sync_ptr), sync_bytes, _P(stream)))


def chain_status(sync_ptr):
    """The sync buffer's status word (0: every barrier wait completed), cleared."""
    v = _U32(0)
    _check(load().mimg_chain_status(_P(sync_ptr), ctypes.byref(v)))
    return int(v.value)


def linear_a8_chain_dev(phases, sync_ptr, sync_bytes, stream):
    """One launch for a chain of one-row grouped products, bit for bit the
    linear_a8_group_dev calls in order (rows 1, block 256). phases: a list of
    (weights, x_ptr, bias_ptrs or None, y_ptrs); raises NotHandled where the
    chain kernel does not apply."""
    arr = (_ChainPhase * len(phases))()
    for i, (weights, x_ptr, bias_ptrs, y_ptrs) in enumerate(phases):
        ph = arr[i]
        ph.x = x_ptr
        ph.count = len(weights)
        for j, w in enumerate(weights):
            ph.w[j] = w.handle
            ph.y[j] = y_ptrs[j]
            ph.bias[j] = bias_ptrs[j] if bias_ptrs and bias_ptrs[j] else None
    _check(load().mimg_linear_a8_chain_dev(ctypes.cast(arr, _P), len(phases), _P(sync_ptr), sync_bytes, _P(stream)))


def _groups(groups):
    arr = (_ChainPhase * len(groups))()
    for i, (weights, x_ptr, bias_ptrs, y_ptrs) in enumerate(groups):
        ph = arr[i]
        ph.x = x_ptr
        ph.count = len(weights)
        for j, w in enumerate(weights):
            ph.w[j] = w.handle
            ph.y[j] = y_ptrs[j]
            ph.bias[j] = bias_ptrs[j] if bias_ptrs and bias_ptrs[j] else None
    return arr


def linear_a8_set_workspace_bytes(groups):
    """Workspace bytes of linear_a8_set_dev for these groups."""
    v = _U64(0)
    arr = _groups(groups)
    _check(load().mimg_linear_a8_set_workspace_bytes(ctypes.cast(arr, _P), len(groups), ctypes.byref(v)))
    return int(v.value)


def linear_a8_set_dev(groups, ws_ptr, ws_bytes, stream):
    """Independent one-row grouped products (rows 1, block 256) in one
    quantize launch and one product launch, bit for bit the
    linear_a8_group_dev calls. groups: a list of (weights, x_ptr, bias_ptrs
    or None, y_ptrs); raises NotHandled where the set kernel does not apply."""
    arr = _groups(groups)
    _check(load().mimg_linear_a8_set_dev(ctypes.cast(arr, _P), len(groups), _P(ws_ptr), ws_bytes, _P(stream)))


def matmul_a8_quantized_set_dev(groups, ws_ptr, ws_bytes, stream):
    """The product launch of linear_a8_set_dev alone, on rows an earlier set
    call with the same groups quantized into ws."""
    arr = _groups(groups)
    _check(load().mimg_matmul_a8_quantized_set_dev(ctypes.cast(arr, _P), len(groups), _P(ws_ptr), ws_bytes,
                                                   _P(stream)))


def rms_norm_linear_a8_group_dev(weights, x_ptr, resid_ptr, scale_ptr, eps, x_out_ptr, bias_ptrs, y_ptrs, stream):
    """One row: x_out = x + resid, h = rms_norm(x_out) * scale, y_ptrs[i] =
    h . W_i^T (+ bias) in one launch; raises NotHandled where the fused
    kernel does not apply (then call rms_norm_dev and linear_a8_group_dev)."""
    n = len(weights)
    hs = (_U64 * n)(*[w.handle for w in weights])
    ys = (_P * n)(*[_P(p) for p in y_ptrs])
    bs = None if bias_ptrs is None else (_P * n)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_rms_norm_linear_a8_group_dev(hs, n, _P(x_ptr), _o(resid_ptr), _o(scale_ptr), eps,
                                                    _P(x_out_ptr), bs, ys, _P(stream)))


def matmul_a8_quantized_swiglu_dev(weights, x_ptr, rows, bias_ptrs, block, out_ptr, procs, ws_ptr, ws_bytes, stream):
    """gate/up products of 1..8 rows of activations already quantized into
    ws, and swiglu of the two into out [rows, N], in one launch; raises
    NotHandled where the fused launch does not apply (then make the group
    and swiglu calls)."""
    hs = (_U64 * 2)(*[w.handle for w in weights])
    bs = None if bias_ptrs is None else (_P * 2)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_matmul_a8_quantized_swiglu_dev(hs, _P(x_ptr), rows, bs, block, _P(out_ptr), procs, _P(ws_ptr),
                                                      ws_bytes, _P(stream)))


def matmul_a8_quantized_qkv_rope_kv_dev(weights, x_ptr, rows, bias_ptrs, block, q_ptr, pos_ptr, cidx_ptr,
                                        inv_freq_ptr, heads, kv_heads, d, rotary, interleaved, context, kc_ptr,
                                        vc_ptr, f16, ws_ptr, ws_bytes, stream):
    """q, k, v products of activations already quantized into ws, rope and
    the cache scatter (4..8 rows); raises NotHandled where it does not apply
    (then make the group call and rope_kv_dev)."""
    hs = (_U64 * 3)(*[w.handle for w in weights])
    bs = None if bias_ptrs is None else (_P * 3)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_matmul_a8_quantized_qkv_rope_kv_dev(hs, _P(x_ptr), rows, bs, block, _P(q_ptr), _P(pos_ptr),
                                                           _P(cidx_ptr), _P(inv_freq_ptr), heads, kv_heads, d, rotary,
                                                           int(interleaved), context, _P(kc_ptr), _P(vc_ptr), int(f16),
                                                           _P(ws_ptr), ws_bytes, _P(stream)))


def rms_norm_qkv_rope_kv_dev(weights, x_ptr, resid_ptr, scale_ptr, eps, x_out_ptr, bias_ptrs, q_ptr, pos_ptr,
                             cidx_ptr, inv_freq_ptr, heads, kv_heads, d, rotary, interleaved, context, kc_ptr, vc_ptr,
                             f16, stream):
    """One row: rms_norm_linear_a8_group_dev on (q, k, v) then rope_kv_dev,
    in one launch (k and v go to the caches only); raises NotHandled where
    the fused launch does not apply (then make the two calls)."""
    hs = (_U64 * 3)(*[w.handle for w in weights])
    bs = None if bias_ptrs is None else (_P * 3)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_rms_norm_qkv_rope_kv_dev(hs, _P(x_ptr), _o(resid_ptr), _o(scale_ptr), eps, _P(x_out_ptr), bs,
                                                _P(q_ptr), _P(pos_ptr), _P(cidx_ptr), _P(inv_freq_ptr), heads,
                                                kv_heads, d, rotary, int(interleaved), context, _P(kc_ptr),
                                                _P(vc_ptr), int(f16), _P(stream)))


def matmul_a8_quantized_dev(w, x_ptr, rows, bias_ptr, block, y_ptr, ws_ptr, ws_bytes, stream):
    _check(load().mimg_matmul_a8_quantized_dev(w.handle, _P(x_ptr), rows, _P(bias_ptr) if bias_ptr else None,
                                               block, _P(y_ptr), _P(ws_ptr), ws_bytes, _P(stream)))


def matmul_a8_quantized_q8_0_tiled_dev(w, x_ptr, rows, bias_ptr, y_ptr, ws_ptr, ws_bytes, stream):
    """Q8_0 x activations quantized in blocks of 32 on the int8 matrix cores:
    one float chain of exact block sums per output, a tolerance claim (not
    the reference's lane order; the default entry points keep that)."""
    _check(load().mimg_matmul_a8_quantized_q8_0_tiled_dev(w.handle, _P(x_ptr), rows,
                                                          _P(bias_ptr) if bias_ptr else None, _P(y_ptr),
                                                          _P(ws_ptr), ws_bytes, _P(stream)))


def matmul_a8_quantized_b32_tiled_dev(w, x_ptr, rows, bias_ptr, y_ptr, ws_ptr, ws_bytes, stream):
    """Q8_0, Q4_K or Q6_K x activations quantized in blocks of 32 on the
    int8 matrix cores (each weight byte read once per tile of rows): one
    float chain per weight block, a tolerance claim (not the reference's
    lane order; the default entry points keep that)."""
    _check(load().mimg_matmul_a8_quantized_b32_tiled_dev(w.handle, _P(x_ptr), rows,
                                                         _P(bias_ptr) if bias_ptr else None, _P(y_ptr),
                                                         _P(ws_ptr), ws_bytes, _P(stream)))


def matmul_a8_quantized_group_dev(weights, x_ptr, rows, bias_ptrs, block, y_ptrs, ws_ptr, ws_bytes, stream):
    n = len(weights)
    hs = (_U64 * n)(*[w.handle for w in weights])
    ys = (_P * n)(*[_P(p) for p in y_ptrs])
    bs = None if bias_ptrs is None else (_P * n)(*[_P(p) if p else None for p in bias_ptrs])
    _check(load().mimg_matmul_a8_quantized_group_dev(hs, n, _P(x_ptr), rows, bs, block, ys, _P(ws_ptr), ws_bytes,
                                                     _P(stream)))


def rms_norm_quant_dev(x_ptr, resid_ptr, scale_ptr, eps, rows, n, y_ptr, block, ws_ptr, ws_bytes, stream):
    _check(load().mimg_rms_norm_quant_dev(_P(x_ptr), _o(resid_ptr), _o(scale_ptr), eps, rows, n, _P(y_ptr), block,
                                          _P(ws_ptr), ws_bytes, _P(stream)))


def swiglu_quant_dev(g_ptr, u_ptr, out_ptr, rows, n, procs, block, ws_ptr, ws_bytes, stream):
    _check(load().mimg_swiglu_quant_dev(_P(g_ptr), _P(u_ptr), _P(out_ptr), rows, n, procs, block, _P(ws_ptr),
                                        ws_bytes, _P(stream)))


def rope_kv_dev(q_ptr, k_ptr, v_ptr, pos_ptr, cidx_ptr, inv_freq_ptr, T, heads, kv_heads, d, rotary, interleaved,
                context, kc_ptr, vc_ptr, f16, stream):
    _check(load().mimg_rope_kv_dev(_P(q_ptr), _P(k_ptr), _P(v_ptr), _P(pos_ptr), _P(cidx_ptr), _P(inv_freq_ptr), T,
                                   heads, kv_heads, d, rotary, int(interleaved), context, _P(kc_ptr), _P(vc_ptr),
                                   int(f16), _P(stream)))


def linear_f32_dev(w, x_ptr, rows, bias_ptr, y_ptr, stream):
    _check(load().mimg_linear_f32_dev(w.handle, _P(x_ptr), rows, _P(bias_ptr) if bias_ptr else None,
                                      _P(y_ptr), _P(stream)))


def linear_f32_mfma_dev(w, x_ptr, rows, bias_ptr, y_ptr, stream):
    """dequant_matmul.v1 on the fp32 matrix cores (mimg_linear_f32_mfma_dev):
    within (K+1)*2^-24*sum|x w| of the exact product, not the reference's
    float order."""
    _check(load().mimg_linear_f32_mfma_dev(w.handle, _P(x_ptr), rows, _P(bias_ptr) if bias_ptr else None,
                                           _P(y_ptr), _P(stream)))


def dequantize_dev(dt, src_ptr, nbytes, dst_ptr, n, stream):
    _check(load().mimg_dequantize_dev(dt, _P(src_ptr), nbytes, _P(dst_ptr), n, _P(stream)))


def quantize_dev(dt, x_ptr, n, dst_ptr, dst_bytes, stream):
    """Encodes n f32 values into blocks of dt on the GPU (the reference
    Quantize for Q8_0, quant.go:165-228; this repository's encoder for
    Q4_K/Q6_K, which the reference lacks)."""
    _check(load().mimg_quantize_dev(dt, _P(x_ptr), n, _P(dst_ptr), dst_bytes, _P(stream)))


def synthetic_normal_dev(seed, std, dst_ptr, n, stream):
    _check(load().mimg_synthetic_normal_dev(seed, std, _P(dst_ptr), n, _P(stream)))


def _o(ptr):
    return _P(ptr) if ptr else None


# ---- the other ops of a decoder step (device pointers, as above) ----------

def embedding_dev(table, ids_ptr, T, out_ptr, stream):
    _check(load().mimg_embedding_dev(table.handle, _P(ids_ptr), T, _P(out_ptr), _P(stream)))


def rms_norm_dev(x_ptr, resid_ptr, scale_ptr, eps, rows, n, y_ptr, stream):
    _check(load().mimg_rms_norm_dev(_P(x_ptr), _o(resid_ptr), _o(scale_ptr), eps, rows, n, _P(y_ptr), _P(stream)))


def rope_dev(x_ptr, pos_ptr, inv_freq_ptr, T, heads, d, rotary, interleaved, stream):
    _check(load().mimg_rope_dev(_P(x_ptr), _P(pos_ptr), _P(inv_freq_ptr), T, heads, d, rotary, int(interleaved),
                                _P(stream)))


def vcache_len(context):
    """Keys a value cache of `context` entries holds: the value cache is
    blocked by eight keys, [kv_heads][ceil(context/8)][d][8]."""
    return (int(context) + 7) // 8 * 8


def vcache_elems(kv_heads, context, d):
    """Elements of a blocked value cache (mimg_vcache_elems)."""
    return int(load().mimg_vcache_elems(kv_heads, context, d))


def pack_vcache(v):
    """A value cache [kv_heads, context, d] (numpy) in the library's blocked
    layout [kv_heads, ceil(context/8), d, 8] (entries past context zero)."""
    hk, c, d = v.shape
    cp = vcache_len(c)
    pad = np.zeros((hk, cp, d), v.dtype)
    pad[:, :c] = v
    return np.ascontiguousarray(pad.reshape(hk, cp // 8, 8, d).transpose(0, 1, 3, 2))


def unpack_vcache(b, kv_heads, context, d):
    """The inverse of pack_vcache, from the raw blocked values."""
    cp = vcache_len(context)
    return np.ascontiguousarray(b.reshape(kv_heads, cp // 8, d, 8).transpose(0, 1, 3, 2).reshape(kv_heads, cp, d)[:, :context])


def kv_store_dev(k_ptr, v_ptr, pos_ptr, T, kv_heads, d, context, kc_ptr, vc_ptr, f16, stream):
    _check(load().mimg_kv_store_dev(_P(k_ptr), _P(v_ptr), _P(pos_ptr), T, kv_heads, d, context, _P(kc_ptr),
                                    _P(vc_ptr), int(f16), _P(stream)))


def attention_workspace_bytes(T, heads, max_keys):
    return int(load().mimg_attention_workspace_bytes(T, heads, max_keys))


def attention_dev(q_ptr, kc_ptr, vc_ptr, kend_ptr, kstart_ptr, T, heads, kv_heads, d, context, max_keys, f16,
                  out_ptr, ws_ptr, ws_bytes, stream):
    _check(load().mimg_attention_dev(_P(q_ptr), _P(kc_ptr), _P(vc_ptr), _P(kend_ptr), _o(kstart_ptr), T, heads,
                                     kv_heads, d, context, max_keys, int(f16), _P(out_ptr), _o(ws_ptr), ws_bytes,
                                     _P(stream)))


def greedy_advance_dev(chosen_ptr, ids_ptr, pos_ptr, cidx_ptr, out_ptr, count_ptr, cap, n, stream):
    _check(load().mimg_greedy_advance_dev(_P(chosen_ptr), _P(ids_ptr), _P(pos_ptr), _o(cidx_ptr), _P(out_ptr),
                                          _P(count_ptr), cap, n, _P(stream)))


def swiglu_dev(g_ptr, u_ptr, out_ptr, n, procs, stream):
    """procs: the reference's GOMAXPROCS, which fixes its piece split."""
    _check(load().mimg_swiglu_dev(_P(g_ptr), _P(u_ptr), _P(out_ptr), n, procs, _P(stream)))


def argmax_dev(x_ptr, rows, n, out_ptr, stream):
    _check(load().mimg_argmax_dev(_P(x_ptr), rows, n, _P(out_ptr), _P(stream)))


def row_bytes(dt, k):
    return k // BLOCK_ELEMS[dt] * BLOCK_BYTES[dt]


def stream_read_dev(ranges, per_thread, sink_ptr, stream):
    """A plain streaming read of up to eight (device pointer, bytes) ranges
    in one launch (mimg_stream_read_dev): the HBM read ceiling."""
    n = len(ranges)
    ps = (_P * n)(*[_P(p) for p, _ in ranges])
    ls = (_U64 * n)(*[b for _, b in ranges])
    _check(load().mimg_stream_read_dev(ps, ls, n, per_thread, _P(sink_ptr), _P(stream)))
