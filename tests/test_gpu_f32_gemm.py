"""dequant_matmul.v1 for prefill rows on the fp32 matrix cores
(mimg_linear_f32_mfma_dev). The summation order is not the reference's, so
the check is the spec's bound for dequant_matmul.v1 (reference
spec/stdlib.md:230-246): |y - exact| <= (K+1) u sum_k |x_k w_k|, u = 2^-24,
with the exact product of the decoded weights (mim.Dequantize, bit for bit
by the oracle) taken in float64, whose own error (K 2^-53 sum|x w|) is 2^-29
of the bound; plus one rounding of the bias addition, as the reference adds
the bias to the finished sum."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 66, 67, 64
U = 2.0 ** -24


def _run(gpu, W, x, bias=None):
    import hiprt

    rows = x.shape[0]
    xd = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    yd = hiprt.DeviceBuffer(rows * W.n * 4)
    bd = None if bias is None else hiprt.DeviceBuffer.from_array(bias)
    s = hiprt.Stream()
    gpu.linear_f32_mfma_dev(W, xd.ptr, rows, bd.ptr if bd else None, yd.ptr, s.handle)
    s.sync()
    return yd.download(np.float32).reshape(rows, W.n)


def _bound_check(oracle, dt, wb, x, n, k, got, bias=None):
    wd = oracle.dequantize(dt, wb, n * k).reshape(n, k).astype(np.float64)
    x64 = x.astype(np.float64)
    exact = x64 @ wd.T
    mag = np.abs(x64) @ np.abs(wd).T
    tol = (k + 1) * U * mag
    if bias is not None:
        exact = exact + bias.astype(np.float64)
        tol = tol + 2 * U * np.abs(exact)
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(tol, 1e-300)))
    assert np.all(err <= tol), f"worst error {worst:.3f} of the bound"
    return worst


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,n,k", [(1, 5, 256), (7, 130, 512), (64, 128, 256), (130, 257, 1024),
                                      (257, 64, 4096), (300, 129, 2048),
                                      (250, 16384, 256)])  # 256 tiles of 128 rows: the 128-row tiling
def test_f32_mfma_within_spec_bound(gpu, oracle, dt, rows, n, k):
    wb = oracle.synthetic_weight(dt, n, k, seed=rows + n)
    x = oracle.synthetic_acts(rows, k, seed=k)
    W = gpu.Weight(wb, dt, n, k)
    got = _run(gpu, W, x)
    W.release()
    _bound_check(oracle, dt, wb, x, n, k, got)


@pytest.mark.parametrize("rows,n,k", [(3, 33, 96), (130, 70, 160), (128, 128, 4096)])
def test_f32_mfma_q8_0_within_spec_bound(gpu, oracle, rows, n, k):
    wb = oracle.synthetic_weight(Q8_0, n, k, seed=n)
    x = oracle.synthetic_acts(rows, k, seed=rows)
    W = gpu.Weight(wb, Q8_0, n, k)
    got = _run(gpu, W, x)
    W.release()
    _bound_check(oracle, Q8_0, wb, x, n, k, got)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_f32_mfma_bias_and_near_the_exact_path(gpu, oracle, dt):
    """With a bias; and the reference-order path (mimg_dequant_matmul) on the
    same inputs is within the same bound, so the two differ by at most
    twice it."""
    rows, n, k = 40, 96, 1024
    wb = oracle.synthetic_weight(dt, n, k, seed=5)
    x = oracle.synthetic_acts(rows, k, seed=6)
    bias = np.random.default_rng(7).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    got = _run(gpu, W, x, bias)
    ref = gpu.dequant_matmul(W, x, bias=bias)
    W.release()
    _bound_check(oracle, dt, wb, x, n, k, got, bias)
    _bound_check(oracle, dt, wb, x, n, k, ref, bias)


def test_f32_mfma_non_finite_inputs_propagate(gpu, oracle):
    """A NaN activation makes its row NaN, an infinite block scale its weight
    row non-finite, as in the reference order (mimg_dequant_matmul)."""
    rows, n, k = 20, 40, 512
    w = bytearray(oracle.synthetic_weight(Q4_K, n, k, seed=2).tobytes())
    rb = len(w) // n
    w[rb * 3 + 0], w[rb * 3 + 1] = 0x00, 0x7C  # row 3, block 0: d = inf
    w = np.frombuffer(bytes(w), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=3)
    x[5, 100] = np.nan
    W = gpu.Weight(w, Q4_K, n, k)
    got = _run(gpu, W, x)
    ref = gpu.dequant_matmul(W, x)
    W.release()
    assert np.isnan(got[5]).all()
    assert np.array_equal(np.isfinite(got), np.isfinite(ref))
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def test_f32_mfma_errors(gpu, oracle):
    import mimg

    wb = oracle.synthetic_weight(Q4_K, 4, 256, seed=1)
    W = gpu.Weight(wb, Q4_K, 4, 256)
    with pytest.raises(mimg.MimgError):
        gpu.linear_f32_mfma_dev(W, 0, 3, None, 0, None)
    gpu.linear_f32_mfma_dev(W, 0, 0, None, 0, None)  # no rows: nothing to do
    W.release()
