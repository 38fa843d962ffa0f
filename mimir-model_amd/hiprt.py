"""Minimal ctypes access to the HIP runtime that libmimg.so links
(/opt/rocm/lib/libamdhip64.so.7): device buffers, copies, streams, events
and stream capture into HIP graphs.

Plumbing for tests and benchmarks. It keeps every GPU call of a process on
one HIP runtime: torch ships its own libamdhip64, and loading both in one
process left torch without a device, so GPU code here does not use torch.
"""
import ctypes
import os

import numpy as np

_rt = None


def rt():
    global _rt
    if _rt is None:
        path = os.environ.get("MIMG_HIP_RUNTIME", "/opt/rocm/lib/libamdhip64.so.7")
        L = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        P, I, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        PP = ctypes.POINTER(ctypes.c_void_p)
        sigs = {
            "hipMalloc": [PP, SZ],
            "hipFree": [P],
            "hipMemcpy": [P, P, SZ, I],
            "hipMemcpyAsync": [P, P, SZ, I, P],
            "hipMemset": [P, I, SZ],
            "hipMemsetAsync": [P, I, SZ, P],
            "hipDeviceSynchronize": [],
            "hipSetDevice": [I],
            "hipStreamCreateWithFlags": [PP, ctypes.c_uint],
            "hipStreamDestroy": [P],
            "hipStreamSynchronize": [P],
            "hipEventCreate": [PP],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
            "hipStreamBeginCapture": [P, I],
            "hipStreamEndCapture": [P, PP],
            "hipGraphInstantiate": [PP, P, PP, ctypes.c_char_p, SZ],
            "hipGraphLaunch": [P, P],
            "hipGraphExecDestroy": [P],
            "hipGraphDestroy": [P],
            "hipGetErrorString": [I],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else I
        _rt = L
    return _rt


H2D, D2H, D2D = 1, 2, 3


def check(rc, what=""):
    if rc != 0:
        raise RuntimeError(f"HIP error {rc} in {what}: {rt().hipGetErrorString(rc).decode()}")


class DeviceBuffer:
    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, stream=None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(rt().hipMemcpy(ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D), "H2D")

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        check(rt().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr + offset), out.nbytes, D2H), "D2H")
        return out

    def zero(self):
        """Zero-fills the buffer and waits for it: hipMemset runs on the null
        stream, which the library's non-blocking streams do not wait for, so
        a kernel enqueued right after could otherwise race with the fill."""
        check(rt().hipMemset(ctypes.c_void_p(self.ptr), 0, self.nbytes), "hipMemset")
        check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")

    def free(self):
        if self.ptr:
            check(rt().hipFree(ctypes.c_void_p(self.ptr)), "hipFree")
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(rt().hipStreamCreateWithFlags(ctypes.byref(s), 1), "hipStreamCreate")  # non-blocking
        self.handle = s.value

    def sync(self):
        check(rt().hipStreamSynchronize(ctypes.c_void_p(self.handle)), "hipStreamSynchronize")

    def destroy(self):
        if self.handle:
            check(rt().hipStreamDestroy(ctypes.c_void_p(self.handle)), "hipStreamDestroy")
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream):
        check(rt().hipEventRecord(ctypes.c_void_p(self.handle), ctypes.c_void_p(stream.handle)), "hipEventRecord")

    def sync(self):
        check(rt().hipEventSynchronize(ctypes.c_void_p(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(rt().hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(self.handle), ctypes.c_void_p(end.handle)), "hipEventElapsedTime")
        return ms.value

    def destroy(self):
        if self.handle:
            check(rt().hipEventDestroy(ctypes.c_void_p(self.handle)), "hipEventDestroy")
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Graph:
    """Captures the work a callable enqueues on `stream` into a HIP graph."""

    def __init__(self, stream, fn):
        check(rt().hipStreamBeginCapture(ctypes.c_void_p(stream.handle), 1), "hipStreamBeginCapture")  # thread-local
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            rc = rt().hipStreamEndCapture(ctypes.c_void_p(stream.handle), ctypes.byref(g))
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        ge = ctypes.c_void_p()
        check(rt().hipGraphInstantiate(ctypes.byref(ge), ctypes.c_void_p(self.graph), None, None, 0), "hipGraphInstantiate")
        self.exec = ge.value

    def launch(self, stream):
        check(rt().hipGraphLaunch(ctypes.c_void_p(self.exec), ctypes.c_void_p(stream.handle)), "hipGraphLaunch")

    def destroy(self):
        """Frees the executable graph and the graph (a replay still in flight
        finishes first: hipGraphExecDestroy waits for it)."""
        if getattr(self, "exec", 0):
            check(rt().hipGraphExecDestroy(ctypes.c_void_p(self.exec)), "hipGraphExecDestroy")
            self.exec = 0
        if getattr(self, "graph", 0):
            check(rt().hipGraphDestroy(ctypes.c_void_p(self.graph)), "hipGraphDestroy")
            self.graph = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def device_sync():
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
