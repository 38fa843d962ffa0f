"""Concurrent callers of the C ABI.

The reference runs sessions of one Program concurrently: Session.Run may be
called from several goroutines, each running the fast paths on the same
weights (reference interp/pool.go:30-40, interp/interp.go:409-523). Here
four threads call libmimg at once (ctypes releases the GIL for the call),
on weights they share and weights of their own, through the host-memory
entry point (the calling thread's own stream and buffers) and the device
entry points (each thread's own stream). Every result must equal the
oracle's, bit for bit; a thread stops at its first mismatch or error."""
import ctypes
import os
import subprocess
import sys
import threading
import time

import numpy as np
import pytest

from test_gpu_parity import bits_equal, first_diff

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 66, 67
MIMG_ERR_HANDLE = -4


def _dev_product(gpu, hiprt, w, x, stream):
    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(x)
    wsb = gpu.a8_workspace_bytes(rows, k)
    ws = hiprt.DeviceBuffer(wsb)
    y = hiprt.DeviceBuffer(rows * w.n * 4)
    gpu.linear_a8_dev(w, xd.ptr, rows, None, 256, y.ptr, ws.ptr, wsb, stream.handle)
    stream.sync()
    return y.download(np.float32).reshape(rows, w.n)


def test_four_threads_shared_and_own_weights(gpu, oracle):
    import hiprt

    k = 2048
    shared_wb = oracle.synthetic_weight(Q4_K, 512, k, seed=40)
    shared = gpu.Weight(shared_wb, Q4_K, 512, k)
    own_wb = [oracle.synthetic_weight(Q6_K, 192 + 64 * i, k, seed=41 + i) for i in range(4)]
    own = [gpu.Weight(wb, Q6_K, 192 + 64 * i, k) for i, wb in enumerate(own_wb)]
    # 1 row (GEMV), 3 rows (pair GEMV), 6 rows (matrix-core GEMV), 40 rows (GEMM)
    xs = [oracle.synthetic_acts(r, k, seed=50 + i) for i, r in enumerate((1, 3, 6, 40))]
    want_shared = [oracle.linear_a8(x, shared_wb, Q4_K, 512, k, block=256, threads=8) for x in xs]
    want_own = [oracle.linear_a8(x, own_wb[i], Q6_K, own[i].n, k, block=256, threads=8) for i, x in enumerate(xs)]
    errors = []
    start = threading.Barrier(4)

    def worker(i):
        try:
            stream = hiprt.Stream()
            start.wait()
            for it in range(12):
                for w, want in ((shared, want_shared[i]), (own[i], want_own[i])):
                    if it % 2 == 0:
                        got = gpu.dequant_matmul_a8(w, xs[i], block=256)
                    else:
                        got = _dev_product(gpu, hiprt, w, xs[i], stream)
                    if not bits_equal(got, want):
                        errors.append(f"thread {i} iteration {it} n={w.n}: {first_diff(got, want)}")
                        return
            stream.destroy()
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
        assert not t.is_alive(), "a thread did not finish"
    shared.release()
    for w in own:
        w.release()
    assert not errors, errors


def test_release_while_other_threads_call(gpu, oracle):
    """One thread drops the last reference of a weight while three others
    are calling it. Calls that looked the handle up before the release run
    to the end on the live weight and give the right bits; calls that start
    after it report an unknown handle; no call fails otherwise."""
    lib = gpu.load()
    n, k = 1024, 4096
    wb = np.ascontiguousarray(oracle.synthetic_weight(Q4_K, n, k, seed=60))
    x = oracle.synthetic_acts(8, k, seed=61)
    want = oracle.linear_a8(x, wb, Q4_K, n, k, block=256, threads=8)
    h = ctypes.c_uint64()
    assert lib.mimg_register_weight(wb.ctypes.data, wb.size, Q4_K, n, k, ctypes.byref(h)) == 0
    handle = h.value
    ok_calls, errors = [], []
    go, released = threading.Event(), threading.Event()

    def caller(i):
        y = np.empty((8, n), np.float32)
        go.wait()
        t_end = time.time() + 60
        while time.time() < t_end:
            rc = lib.mimg_dequant_matmul_a8(handle, x.ctypes.data, 8, None, 256, y.ctypes.data)
            if rc == MIMG_ERR_HANDLE:
                if not released.is_set() and not release_started.is_set():
                    errors.append(f"thread {i}: unknown handle before the release")
                return
            if rc != 0:
                errors.append(f"thread {i}: rc {rc}: {lib.mimg_last_error().decode()}")
                return
            if not bits_equal(y, want):
                errors.append(f"thread {i}: {first_diff(y, want)}")
                return
            ok_calls.append(i)
        errors.append(f"thread {i}: the handle outlived its release")

    release_started = threading.Event()
    threads = [threading.Thread(target=caller, args=(i,)) for i in range(3)]
    for t in threads:
        t.start()
    go.set()
    t0 = time.time()
    while len(ok_calls) < 30 and time.time() - t0 < 30 and not errors:
        time.sleep(0.001)
    release_started.set()
    assert lib.mimg_release_weight(handle) == 0
    released.set()
    for t in threads:
        t.join(timeout=120)
        assert not t.is_alive(), "a caller did not finish"
    assert not errors, errors
    assert len(ok_calls) >= 30, "too few calls ran before the release"
    assert lib.mimg_release_weight(handle) == MIMG_ERR_HANDLE


_SHUTDOWN_SCRIPT = r"""
import ctypes, sys
import numpy as np
sys.path[:0] = sys.argv[1:3]
import mimg, mimref
lib = mimg.load()
n, k = 128, 1024
wb = np.ascontiguousarray(mimref.synthetic_weight(66, n, k, seed=70))
x = mimref.synthetic_acts(2, k, seed=71)
want = mimref.linear_a8(x, wb, 66, n, k, block=256)
sec = np.concatenate([np.zeros(4096, np.uint8), wb])
for rnd in range(2):
    assert lib.mimg_init(0) == 0, rnd
    base = ctypes.c_void_p()
    assert lib.mimg_upload_weights(sec.ctypes.data, sec.size, ctypes.byref(base)) == 0
    h = ctypes.c_uint64()
    assert lib.mimg_register_weight_view(ctypes.c_void_p(base.value + 4096), wb.size, 66, n, k, ctypes.byref(h)) == 0
    h2 = ctypes.c_uint64()
    assert lib.mimg_register_weight(wb.ctypes.data, wb.size, 66, n, k, ctypes.byref(h2)) == 0
    for hh in (h.value, h2.value):
        y = np.empty((2, n), np.float32)
        assert lib.mimg_dequant_matmul_a8(hh, x.ctypes.data, 2, None, 256, y.ctypes.data) == 0
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (rnd, hh)
    lib.mimg_shutdown()  # frees the section once, the view's flags, the copy
    assert lib.mimg_release_weight(h.value) < 0  # not initialised any more
print("shutdown-reinit ok")
"""


def test_shutdown_with_views_then_reinit(gpu):
    """A weights section with a view and a registered copy, then
    mimg_shutdown (the section freed once, the view's bytes not freed on
    their own) and mimg_init again, twice, in a process of its own (the
    shutdown frees every registration of the process)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _SHUTDOWN_SCRIPT, os.path.join(root, "mimir-model_amd"),
                        os.path.join(root, "oracle")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "shutdown-reinit ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
