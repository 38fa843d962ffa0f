"""ctypes binding of liboracle (libmimref.so), the CPU restatement of the
reference numerics.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product (libmimg.so and its
wrapper) never imports this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MIMREF_LIB") or os.path.join(HERE, "libmimref.so")

F32, Q8_0, Q4_K, Q6_K = 1, 64, 66, 67
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210}

_lib = None


def build():
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        U32 = ctypes.c_uint32
        sigs = {
            "mref_f16_to_f32": (F, [ctypes.c_uint16]),
            "mref_f16_to_f32_n": (None, [P, P, I64]),
            "mref_f32_to_f16": (ctypes.c_uint16, [F]),
            "mref_row_bytes": (I64, [U32, I64]),
            "mref_dequantize": (I, [U32, P, I64, P, I64]),
            "mref_quantize": (I, [U32, P, I64, P, I64]),
            "mref_quantize_act": (I, [P, I64, I, P, P, P, P, P]),
            "mref_dot_q4k_a8k": (I, [P, P, P, P, I64, P]),
            "mref_dot_q6k_a8k": (I, [P, P, P, I64, P]),
            "mref_dot_q8_0_a8": (I, [P, P, P, I64, P]),
            "mref_dot_q4k_a8": (I, [P, P, P, P, I64, P]),
            "mref_dot_q6k_a8": (I, [P, P, P, P, I64, P]),
            "mref_dot_f32": (F, [P, P, I64]),
            "mref_dot_q4k_f32": (F, [P, P, I64]),
            "mref_dot_q6k_f32": (F, [P, P, I64]),
            "mref_dot_q8_0_f32": (F, [P, P, I64]),
            "mref_linear_a8": (I, [P, I64, P, U32, I64, I64, P, I, P, I]),
            "mref_linear_f32": (I, [P, I64, P, U32, I64, I64, P, P, I]),
            "mref_fmaf": (F, [F, F, F]),
            "mref_expsum_f32": (F, [P, I64, F]),
            "mref_scores": (None, [P, P, P, I64, I, F, P]),
            "mref_attend_row": (None, [P, P, P, P, P, I64, I, F, P, P]),
            "mref_attention": (I, [P, P, P, P, P, I64, I, I, I, I64, I, P, I]),
            "mref_silu_mul": (None, [P, P, P, I64, I]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(dt, k):
    return int(lib().mref_row_bytes(dt, k))


def f16_to_f32(h):
    """f16 bits (array) to float32, bits preserved (signalling NaNs too)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.size, np.float32)
    lib().mref_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def dequantize(dt, raw, n):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib().mref_dequantize(dt, _p(raw), raw.size, _p(out), n)
    if rc != 0:
        raise ValueError(f"mref_dequantize: code {rc}")
    return out


def quantize(dt, x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    nbytes = x.size // BLOCK_ELEMS[dt] * BLOCK_BYTES[dt]
    out = np.empty(nbytes, dtype=np.uint8)
    rc = lib().mref_quantize(dt, _p(x), x.size, _p(out), nbytes)
    if rc != 0:
        raise ValueError(f"mref_quantize: code {rc}")
    return out


class Act:
    """One row of 8-bit activations (reference Q8, internal/kernels/q8.go:30-40)."""

    def __init__(self, x, block):
        x = np.ascontiguousarray(x, dtype=np.float32)
        k = x.size
        self.k, self.block = k, block
        self.q = np.zeros(k, np.int8)
        self.d = np.zeros(k // 32, np.float32)
        self.xs = np.zeros(k // 32, np.int16)
        self.m32 = np.zeros(k // 2, np.int16)
        self.dbs = np.zeros(k // 32, np.float32)
        self.ok = bool(lib().mref_quantize_act(_p(x), k, block, _p(self.q), _p(self.d), _p(self.xs), _p(self.m32), _p(self.dbs)))


def dot_a8(dt, row, act):
    """The 8-bit dot product of one weight row with one Act (None if refused)."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = ctypes.c_float()
    L = lib()
    if act.block == 256 and dt == Q4_K:
        ok = L.mref_dot_q4k_a8k(_p(row), _p(act.q), _p(act.d), _p(act.xs), act.k // 256, ctypes.byref(out))
    elif act.block == 256 and dt == Q6_K:
        ok = L.mref_dot_q6k_a8k(_p(row), _p(act.q), _p(act.d), act.k // 256, ctypes.byref(out))
    elif act.block == 32 and dt == Q8_0:
        ok = L.mref_dot_q8_0_a8(_p(row), _p(act.q), _p(act.d), act.k // 32, ctypes.byref(out))
    elif act.block == 32 and dt == Q4_K:
        ok = L.mref_dot_q4k_a8(_p(row), _p(act.q), _p(act.d), _p(act.dbs), act.k // 256, ctypes.byref(out))
    elif act.block == 32 and dt == Q6_K:
        ok = L.mref_dot_q6k_a8(_p(row), _p(act.q), _p(act.d), _p(act.m32), act.k // 256, ctypes.byref(out))
    else:
        raise ValueError("no 8-bit kernel")
    return np.float32(out.value) if ok else None


def dot_f32(dt, row, x):
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = lib()
    if dt == Q4_K:
        return np.float32(L.mref_dot_q4k_f32(_p(row), _p(x), x.size // 256))
    if dt == Q6_K:
        return np.float32(L.mref_dot_q6k_f32(_p(row), _p(x), x.size // 256))
    if dt == Q8_0:
        return np.float32(L.mref_dot_q8_0_f32(_p(row), _p(x), x.size // 32))
    raise ValueError(dt)


def dot_plain_f32(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return np.float32(lib().mref_dot_f32(_p(a), _p(b), a.size))


def linear_a8(x, w_bytes, dt, n, k, bias=None, block=256, threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    w_bytes = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((x.shape[0], n), np.float32)
    rc = lib().mref_linear_a8(_p(x), x.shape[0], _p(w_bytes), dt, n, k, _p(b), block, _p(y), threads)
    if rc != 0:
        raise ValueError(f"mref_linear_a8: code {rc}")
    return y


def linear_f32(x, w_bytes, dt, n, k, bias=None, threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    w_bytes = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((x.shape[0], n), np.float32)
    rc = lib().mref_linear_f32(_p(x), x.shape[0], _p(w_bytes), dt, n, k, _p(b), _p(y), threads)
    if rc != 0:
        raise ValueError(f"mref_linear_f32: code {rc}")
    return y


def fmaf(a, b, c):
    return np.float32(lib().mref_fmaf(a, b, c))


def synthetic_weight(dt, n, k, seed, scale=0.02):
    """W ~ N(0, scale^2) in f32 from numpy's PCG64 (default_rng(seed)), encoded
    with this repository's encoder (the reference has no Q4_K/Q6_K encoder)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(scale)
    return quantize(dt, w)


def synthetic_acts(rows, k, seed):
    """x ~ N(0, 1) in f32 from numpy's PCG64 (default_rng(seed))."""
    return np.random.default_rng(seed).standard_normal((rows, k), dtype=np.float32)


# ---- decoder ops (interp/fast.go:487-498, 559-751 with attn_amd64.s) ----

def expsum_f32(x, m):
    """ExpSumF32: (exponentials, their sum)."""
    x = np.ascontiguousarray(x, np.float32).copy()
    s = lib().mref_expsum_f32(_p(x), x.size, float(np.float32(m)))
    return x, np.float32(s)


def scores(q, k, scale):
    """ScoresF32 (k f32 [n, d]) or ScoresF16 (k float16 [n, d])."""
    q = np.ascontiguousarray(q, np.float32)
    n, d = k.shape
    out = np.empty(n, np.float32)
    if k.dtype == np.float16:
        k16 = np.ascontiguousarray(k).view(np.uint16)
        lib().mref_scores(_p(q), None, _p(k16), n, d, float(np.float32(scale)), _p(out))
    else:
        k32 = np.ascontiguousarray(k, np.float32)
        lib().mref_scores(_p(q), _p(k32), None, n, d, float(np.float32(scale)), _p(out))
    return out


def attention(q, kc, vc, kend, kstart=None, threads=1):
    """q [T, H, D] f32; kc, vc [Hkv, C, D] float32 or float16; query t sees
    cache entries kstart[t]..kend[t] of its kv head."""
    q = np.ascontiguousarray(q, np.float32)
    T, H, D = q.shape
    Hkv, C, _ = kc.shape
    f16 = kc.dtype == np.float16
    kc = np.ascontiguousarray(kc).view(np.uint16) if f16 else np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc).view(np.uint16) if f16 else np.ascontiguousarray(vc, np.float32)
    ke = np.ascontiguousarray(kend, np.int64)
    ks = None if kstart is None else np.ascontiguousarray(kstart, np.int64)
    out = np.empty_like(q)
    rc = lib().mref_attention(_p(q), _p(kc), _p(vc), _p(ke), _p(ks), T, H, Hkv, D, C, int(f16), _p(out), threads)
    if rc != 0:
        raise ValueError(f"mref_attention: {rc}")
    return out


def silu_mul(a, b, procs):
    """swiglu.v1 with the piece split of GOMAXPROCS = procs."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    lib().mref_silu_mul(_p(a), _p(b), _p(out), a.size, procs)
    return out

