"""mimg_linear_a8_noalloc_dev: the 8-bit product with the library's static
scratch instead of a caller workspace, for callers that cannot allocate. It
must equal mimg_linear_a8_dev bit for bit, on two calls in a row (the second
with a smaller input, so it runs on what the first left in the scratch), and
refuse sizes the scratch cannot hold."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 66, 67, 64


def _with_workspace(gpu, hiprt, w, x, bias, block, stream):
    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(x)
    wsb = gpu.a8_workspace_bytes(rows, k)
    ws = hiprt.DeviceBuffer(wsb)
    y = hiprt.DeviceBuffer(rows * w.n * 4)
    gpu.linear_a8_dev(w, xd.ptr, rows, bias.ptr if bias else None, block, y.ptr, ws.ptr, wsb, stream.handle)
    stream.sync()
    return y.download(np.float32).reshape(rows, w.n)


def _no_alloc(gpu, hiprt, w, x, bias, block, stream):
    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(x)
    y = hiprt.DeviceBuffer(rows * w.n * 4)
    gpu.linear_a8_noalloc_dev(w, xd.ptr, rows, bias.ptr if bias else None, block, y.ptr, stream.handle)
    stream.sync()
    return y.download(np.float32).reshape(rows, w.n)


@pytest.mark.parametrize("dt,block", [(Q4_K, 256), (Q6_K, 256), (Q8_0, 32), (Q4_K, 32)])
def test_no_alloc_equals_workspace_call(gpu, oracle, dt, block):
    import hiprt

    n, k = 700, 4096
    wb = oracle.synthetic_weight(dt, n, k, seed=80 + dt)
    W = gpu.Weight(wb, dt, n, k)
    bias = hiprt.DeviceBuffer.from_array(np.random.default_rng(81).standard_normal(n).astype(np.float32))
    s = hiprt.Stream()
    # 40 rows (the GEMM for blocks of 256), then 3 rows with a refused row
    # (the pair GEMV and the float32 path) on what the first call left
    for rows, seed in ((40, 82), (3, 83)):
        x = oracle.synthetic_acts(rows, k, seed=seed)
        if rows == 3:
            x[1, 77] = np.float32(np.inf)
        want = _with_workspace(gpu, hiprt, W, x, bias, block, s)
        got = _no_alloc(gpu, hiprt, W, x, bias, block, s)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rows, int(np.sum(got != want)))
    W.release()


def test_no_alloc_refuses_what_the_scratch_cannot_hold(gpu, oracle):
    import hiprt

    k = 14336
    W = gpu.Weight(oracle.synthetic_weight(Q6_K, 8, k, seed=84), Q6_K, 8, k)
    cap = int(gpu.load().mimg_noalloc_scratch_bytes())
    rows = 1
    while gpu.a8_workspace_bytes(rows, k) <= cap:
        rows *= 2
    x = hiprt.DeviceBuffer(rows * k * 4)
    y = hiprt.DeviceBuffer(rows * 8 * 4)
    s = hiprt.Stream()
    with pytest.raises(gpu.MimgError) as e:
        gpu.linear_a8_noalloc_dev(W, x.ptr, rows, None, 256, y.ptr, s.handle)
    assert e.value.code == -6 and "scratch" in str(e.value)
    # row counts whose workspace size would overflow 64 bits are refused the
    # same way (the check comes before the size arithmetic; nothing is read)
    for huge in (1 << 62, (1 << 63) - 1, (1 << 64) // k + 1):
        with pytest.raises(gpu.MimgError) as e:
            gpu.linear_a8_noalloc_dev(W, x.ptr, huge, None, 256, y.ptr, s.handle)
        assert e.value.code == -6, huge
    W.release()
