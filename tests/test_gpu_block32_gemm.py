"""Q8_0, Q4_K and Q6_K weights with activation blocks of 32 from 16 rows.

The default entry points (dequant_matmul_a8 with block 32) keep the
reference's eight-lane order of dotQ8_0Q8AVX2 (kernels_amd64.s:1007-1043)
at every row count, so they equal the oracle bit for bit and a row's bits
do not depend on the rows beside it.

mimg_matmul_a8_quantized_q8_0_tiled_dev (Q8_0, gemm_q8_0.hip) and
mimg_matmul_a8_quantized_b32_tiled_dev (Q4_K and Q6_K, gemm_kq_b32.hip; Q8_0
through the former) are the opt-in matrix-core forms (int8 MFMA GEMMs): one
chain of exact block sums, not the reference's lane order, so their claim is
the spec's tolerance for dequant_matmul_a8 (reference spec/stdlib.md:260-275):
    |y - exact| <= (K+2) u (sum_k (|x_k| + s_k) B_k + |bias|) + sum_k s_k |wd_k|
with wd the reference decode of the weights (the oracle's mim.Dequantize,
bit for bit), B_k = |wd_k| for Q8_0 and Q6_K and |d sc_j q_k| + |dmin m_j|
for Q4_K (the two terms of the decode), s_k the largest |x| of k's block of
32 over 127, u = 2^-24, and the exact product taken in float64 (its own error
is ~2^-29 of the bound). Rows the reference refuses (NaN or |x| > 2^60 in
x, a non-finite block scale in w) take its float32 path and must equal the
oracle's bit for bit, NaN and Inf included."""
import numpy as np
import pytest

from test_gpu_parity import bits_equal, first_diff

pytestmark = pytest.mark.gpu

Q8_0 = 64
U = 2.0 ** -24


def tiled(gpu, W, x, bias=None):
    """The opt-in matrix-core Q8_0 product of x (quantized in blocks of 32)."""
    import hiprt

    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    wsb = gpu.a8_workspace_bytes(rows, k)
    ws = hiprt.DeviceBuffer(wsb)
    yd = hiprt.DeviceBuffer(rows * W.n * 4)
    bd = hiprt.DeviceBuffer.from_array(bias) if bias is not None else None
    s = hiprt.Stream()
    gpu.quantize_act_dev(xd.ptr, rows, k, 32, ws.ptr, wsb, s.handle)
    gpu.matmul_a8_quantized_q8_0_tiled_dev(W, xd.ptr, rows, bd.ptr if bd else None, yd.ptr, ws.ptr, wsb, s.handle)
    s.sync()
    y = yd.download(np.float32).reshape(rows, W.n)
    for b in (xd, ws, yd, bd):
        if b is not None:
            b.free()
    return y


def _bound_check(oracle, wb, x, n, k, got, bias=None):
    wd = oracle.dequantize(Q8_0, wb, n * k).reshape(n, k).astype(np.float64)
    x64 = x.astype(np.float64)
    ax = np.abs(x64)
    s = np.repeat(ax.reshape(x.shape[0], -1, 32).max(axis=2) / 127.0, 32, axis=1)
    aw = np.abs(wd)
    exact = x64 @ wd.T
    tol = (k + 2) * U * ((ax + s) @ aw.T) + s @ aw.T
    if bias is not None:
        exact = exact + bias.astype(np.float64)
        tol = tol + (k + 2) * U * np.abs(bias.astype(np.float64))
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(tol, 1e-300)))
    assert np.all(err <= tol), f"worst error {worst:.3f} of the bound"
    return worst


@pytest.mark.parametrize("rows,n,k,with_bias", [(16, 64, 256, False), (130, 300, 1024, True), (257, 129, 2048, False),
                                                (600, 1000, 4096, True), (1030, 4100, 512, False)])
def test_q8_0_gemm_within_a8_bound(gpu, oracle, rows, n, k, with_bias):
    wb = oracle.synthetic_weight(Q8_0, n, k, seed=rows + n)
    x = oracle.synthetic_acts(rows, k, seed=k + 3)
    bias = np.random.default_rng(4).standard_normal(n).astype(np.float32) if with_bias else None
    W = gpu.Weight(wb, Q8_0, n, k)
    got = tiled(gpu, W, x, bias)
    W.release()
    _bound_check(oracle, wb, x, n, k, got, bias)


def test_q8_0_gemm_rows_are_independent(gpu, oracle):
    """Each output depends on its own activation row only: the first 40
    rows give the same bits alone (one tile) as inside 1100 rows."""
    n, k = 700, 2048
    wb = oracle.synthetic_weight(Q8_0, n, k, seed=5)
    x = oracle.synthetic_acts(1100, k, seed=6)
    W = gpu.Weight(wb, Q8_0, n, k)
    many = tiled(gpu, W, x)
    few = tiled(gpu, W, x[:40])
    W.release()
    assert bits_equal(many[:40], few), first_diff(many[:40], few)


def test_q8_0_gemm_refusals_match_the_reference_path(gpu, oracle):
    """A NaN row and a row above 2^60 of x, weight rows with an infinite and
    a NaN block scale: their outputs are the reference's float32 path bit
    for bit (NaN/Inf propagation included); the rest within the bound."""
    n, k, rows = 300, 1024, 70
    wb = bytearray(oracle.synthetic_weight(Q8_0, n, k, seed=7).tobytes())
    rb = len(wb) // n
    wb[rb * 11 + 34 * 3:rb * 11 + 34 * 3 + 2] = b"\x00\x7c"   # +inf scale, row 11
    wb[rb * 200 + 34 * 0:rb * 200 + 2] = b"\x01\x7e"           # NaN scale, row 200
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=8)
    x[3, 5] = np.nan
    x[50, 700] = np.float32(3e19)
    bias = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, Q8_0, n, k)
    assert W.info()[1] == 2
    got = tiled(gpu, W, x, bias)
    W.release()
    want = oracle.linear_a8(x, wb, Q8_0, n, k, bias=bias, block=32, threads=16)
    refused_rows, refused_cols = [3, 50], [11, 200]
    for r in refused_rows:
        assert bits_equal(got[r], want[r]), (r, first_diff(got[r], want[r]))
    for c in refused_cols:
        assert bits_equal(got[:, c], want[:, c]), (c, first_diff(got[:, c], want[:, c]))
    keep_r = np.setdiff1d(np.arange(rows), refused_rows)
    keep_c = np.setdiff1d(np.arange(n), refused_cols)
    wb_keep = np.concatenate([wb[rb * c:rb * (c + 1)] for c in keep_c])
    _bound_check(oracle, wb_keep, x[keep_r], keep_c.size, k, got[np.ix_(keep_r, keep_c)], bias[keep_c])


CFG2_Q8 = [("gate", 14336, 4096, 4), ("down", 4096, 14336, 6)]


@pytest.mark.parametrize("rows", [64, 512, 2048])
@pytest.mark.parametrize("name,n,k,seed", CFG2_Q8, ids=[c[0] for c in CFG2_Q8])
def test_cfg2_q8_0_variant_within_a8_bound(gpu, oracle, name, n, k, seed, rows):
    """BASELINE config 2's Q8_0 variant of gate/up and down at 64, 512 and
    2048 rows (62 MB of weights each): every output row of a spread sample
    of 64 rows within the bound (the float64 check of all rows would take
    minutes on the CPU)."""
    wb = oracle.synthetic_weight(Q8_0, n, k, seed)
    x = oracle.synthetic_acts(rows, k, seed=300 + rows)
    print(f"cfg2 Q8_0 {name} rows {rows}", flush=True)
    W = gpu.Weight(wb, Q8_0, n, k)
    got = tiled(gpu, W, x)
    W.release()
    pick = np.arange(rows) if rows <= 512 else np.unique(np.linspace(0, rows - 1, 256).astype(int))
    _bound_check(oracle, wb, x[pick], n, k, got[pick])


@pytest.mark.parametrize("rows,n,k", [(16, 64, 256), (40, 300, 1024), (130, 77, 2048)])
def test_q8_0_block32_default_path_is_the_lane_order(gpu, oracle, rows, n, k):
    """From 16 rows the default entry point keeps the reference's lane order:
    bit for bit the oracle, and each row alone gives the same bits as inside
    the call (what the matrix-core form above does not promise)."""
    wb = oracle.synthetic_weight(Q8_0, n, k, seed=rows + k)
    x = oracle.synthetic_acts(rows, k, seed=rows)
    bias = np.random.default_rng(rows).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, Q8_0, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=32)
    alone = np.concatenate([gpu.dequant_matmul_a8(W, x[i:i + 1], bias=bias, block=32) for i in (0, rows // 2, rows - 1)])
    W.release()
    want = oracle.linear_a8(x, wb, Q8_0, n, k, bias=bias, block=32, threads=8)
    assert bits_equal(got, want), first_diff(got, want)
    assert bits_equal(alone, got[[0, rows // 2, rows - 1]]), first_diff(alone, got[[0, rows // 2, rows - 1]])


# ------------------------------------------------ Q4_K / Q6_K, blocks of 32

Q4_K, Q6_K = 66, 67


def tiled_b32(gpu, W, x, bias=None):
    """The opt-in matrix-core product with activation blocks of 32."""
    import hiprt

    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    wsb = gpu.a8_workspace_bytes(rows, k)
    ws = hiprt.DeviceBuffer(wsb)
    yd = hiprt.DeviceBuffer(rows * W.n * 4)
    bd = hiprt.DeviceBuffer.from_array(bias) if bias is not None else None
    s = hiprt.Stream()
    gpu.quantize_act_dev(xd.ptr, rows, k, 32, ws.ptr, wsb, s.handle)
    gpu.matmul_a8_quantized_b32_tiled_dev(W, xd.ptr, rows, bd.ptr if bd else None, yd.ptr, ws.ptr, wsb, s.handle)
    s.sync()
    y = yd.download(np.float32).reshape(rows, W.n)
    for b in (xd, ws, yd, bd):
        if b is not None:
            b.free()
    return y


def _q4k_terms(wb, n, k):
    """B_k = |d sc_j q_k| + |dmin m_j| of every element of Q4_K rows (the
    reference's getScaleMinK4, quant.go:272-281, and element order)."""
    nb = n * k // 256
    blk = np.asarray(wb, np.uint8).reshape(nb, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float64)
    s = blk[:, 4:16].astype(np.int64)
    sc, m = np.zeros((nb, 8)), np.zeros((nb, 8))
    for j in range(4):
        sc[:, j], m[:, j] = s[:, j] & 63, s[:, j + 4] & 63
        sc[:, j + 4] = (s[:, j + 8] & 15) | ((s[:, j] >> 6) << 4)
        m[:, j + 4] = (s[:, j + 8] >> 4) | ((s[:, j + 4] >> 6) << 4)
    qs = blk[:, 16:144]
    q = np.empty((nb, 256))
    for c in range(4):
        q[:, 64 * c:64 * c + 32] = qs[:, 32 * c:32 * c + 32] & 15
        q[:, 64 * c + 32:64 * c + 64] = qs[:, 32 * c:32 * c + 32] >> 4
    B = np.abs(d * np.repeat(sc, 32, axis=1) * q) + np.abs(dmin * np.repeat(m, 32, axis=1))
    return B.reshape(n, k)


def _bound_check_kq(oracle, dt, wb, x, n, k, got, bias=None):
    wd = oracle.dequantize(dt, wb, n * k).reshape(n, k).astype(np.float64)
    aw = np.abs(wd)
    B = _q4k_terms(wb, n, k) if dt == Q4_K else aw
    x64 = x.astype(np.float64)
    ax = np.abs(x64)
    s = np.repeat(ax.reshape(x.shape[0], -1, 32).max(axis=2) / 127.0, 32, axis=1)
    exact = x64 @ wd.T
    tol = (k + 2) * U * ((ax + s) @ B.T) + s @ aw.T
    if bias is not None:
        exact = exact + bias.astype(np.float64)
        tol = tol + (k + 2) * U * np.abs(bias.astype(np.float64))
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(tol, 1e-300)))
    assert np.all(err <= tol), f"worst error {worst:.3f} of the bound"
    return worst


def test_q4k_terms_match_the_oracle_test_decode(oracle):
    """The vectorised B_k above equals the per-block restatement the oracle's
    own tolerance test uses (tests/test_oracle.py _wd_terms)."""
    from test_oracle import _wd_terms

    n, k = 3, 1024
    wb = oracle.synthetic_weight(Q4_K, n, k, seed=2)
    B = _q4k_terms(wb, n, k)
    rb = wb.size // n
    for r in range(n):
        _, want = _wd_terms(Q4_K, wb[rb * r:rb * (r + 1)].tobytes(), k, oracle)
        assert np.array_equal(B[r], want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K], ids=["q4_k", "q6_k"])
@pytest.mark.parametrize("rows,n,k,with_bias", [(16, 300, 256, False),     # small-grid 16 x 64 tiles
                                                (130, 8000, 512, True),    # 64 x 64 tiles
                                                (300, 16384, 256, False),  # 128 x 128 tiles
                                                (70, 129, 2048, True), (1030, 200, 1024, False)])
def test_kq_b32_gemm_within_a8_bound(gpu, oracle, dt, rows, n, k, with_bias):
    wb = oracle.synthetic_weight(dt, n, k, seed=rows + n + dt)
    x = oracle.synthetic_acts(rows, k, seed=k + 5)
    bias = np.random.default_rng(4).standard_normal(n).astype(np.float32) if with_bias else None
    W = gpu.Weight(wb, dt, n, k)
    got = tiled_b32(gpu, W, x, bias)
    W.release()
    _bound_check_kq(oracle, dt, wb, x, n, k, got, bias)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K], ids=["q4_k", "q6_k"])
def test_kq_b32_gemm_rows_are_independent(gpu, oracle, dt):
    """The first 40 rows give the same bits alone (the small-grid 16 x 64
    tiles) as inside 1100 rows (64 x 64 tiles)."""
    n, k = 2100, 1024
    wb = oracle.synthetic_weight(dt, n, k, seed=5)
    x = oracle.synthetic_acts(1100, k, seed=6)
    W = gpu.Weight(wb, dt, n, k)
    many = tiled_b32(gpu, W, x)
    few = tiled_b32(gpu, W, x[:40])
    W.release()
    assert bits_equal(many[:40], few), first_diff(many[:40], few)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K], ids=["q4_k", "q6_k"])
def test_kq_b32_gemm_refusals_match_the_reference_path(gpu, oracle, dt):
    """A NaN row and a row above 2^60 of x, weight rows with an infinite and
    a NaN block scale: their outputs are the reference's float32 path bit
    for bit; the rest within the bound."""
    n, k, rows = 300, 1024, 70
    bb, doff = (144, 0) if dt == Q4_K else (210, 208)
    wb = bytearray(oracle.synthetic_weight(dt, n, k, seed=7).tobytes())
    rb = len(wb) // n
    wb[rb * 11 + bb * 2 + doff:rb * 11 + bb * 2 + doff + 2] = b"\x00\x7c"  # +inf d, row 11 block 2
    wb[rb * 200 + doff:rb * 200 + doff + 2] = b"\x01\x7e"                # NaN d, row 200 block 0
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=8)
    x[3, 5] = np.nan
    x[50, 700] = np.float32(3e19)
    bias = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    assert W.info()[1] == 2
    got = tiled_b32(gpu, W, x, bias)
    W.release()
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=32, threads=16)
    refused_rows, refused_cols = [3, 50], [11, 200]
    for r in refused_rows:
        assert bits_equal(got[r], want[r]), (r, first_diff(got[r], want[r]))
    for c in refused_cols:
        assert bits_equal(got[:, c], want[:, c]), (c, first_diff(got[:, c], want[:, c]))
    keep_r = np.setdiff1d(np.arange(rows), refused_rows)
    keep_c = np.setdiff1d(np.arange(n), refused_cols)
    wb_keep = np.concatenate([wb[rb * c:rb * (c + 1)] for c in keep_c])
    _bound_check_kq(oracle, dt, wb_keep, x[keep_r], keep_c.size, k, got[np.ix_(keep_r, keep_c)], bias[keep_c])


CFG2_KQ = [("gate", Q4_K, 14336, 4096, 4), ("down", Q6_K, 4096, 14336, 6)]


@pytest.mark.parametrize("rows", [64, 512])
@pytest.mark.parametrize("name,dt,n,k,seed", CFG2_KQ, ids=[c[0] for c in CFG2_KQ])
def test_cfg2_kquant_blocks_of_32_within_a8_bound(gpu, oracle, name, dt, n, k, seed, rows):
    """BASELINE config 2's gate (Q4_K) and down (Q6_K) with activation
    blocks of 32 (a dequant_matmul_a8.v1 graph) at 64 and 512 rows: a spread
    sample of 64 output rows within the bound."""
    wb = oracle.synthetic_weight(dt, n, k, seed)
    x = oracle.synthetic_acts(rows, k, seed=400 + rows)
    print(f"cfg2 {name} blocks of 32, rows {rows}", flush=True)
    W = gpu.Weight(wb, dt, n, k)
    got = tiled_b32(gpu, W, x)
    W.release()
    pick = np.unique(np.linspace(0, rows - 1, 64).astype(int))
    _bound_check_kq(oracle, dt, wb, x[pick], n, k, got[pick])


@pytest.mark.parametrize("dt,rows,n,k", [(Q8_0, 64, 300, 1024),     # small-grid tiles
                                         (Q8_0, 130, 8000, 512),    # 64 x 64 tiles
                                         (Q6_K, 64, 300, 1024),     # small-grid tiles
                                         (Q6_K, 130, 8000, 512)],   # 64 x 64 tiles
                         ids=["q8_0-small", "q8_0-mid", "q6_k-small", "q6_k-mid"])
def test_block32_gemm_unaligned_weight_view(gpu, oracle, dt, rows, n, k):
    """The same weight bytes as a view 2 bytes past a 16-byte boundary of an
    uploaded weights section (the kernels realign the blocks in LDS) and as
    a 16-byte aligned view (Q8_0: the blocks' offsets as constants): equal
    bits."""
    wb = np.ascontiguousarray(oracle.synthetic_weight(dt, n, k, seed=rows + n + 7)).view(np.uint8).ravel()
    assert wb.size % 16 == 0
    section = gpu.WeightsSection(np.concatenate([wb, np.zeros(18, np.uint8), wb, np.zeros(256, np.uint8)]))
    assert section.ptr % 16 == 0
    x = oracle.synthetic_acts(rows, k, seed=k + 9)
    run = tiled if dt == Q8_0 else tiled_b32
    Wa = section.view(0, wb.size, dt, n, k)
    Wu = section.view(wb.size + 18, wb.size, dt, n, k)
    try:
        ya = run(gpu, Wa, x)
        yu = run(gpu, Wu, x)
    finally:
        Wa.release()
        Wu.release()
        section.free()
    assert bits_equal(ya, yu), first_diff(ya, yu)


def test_kq_b32_gemm_q4k_unaligned_view_not_handled(gpu, oracle):
    """Q4_K blocks are copied as whole 16-byte chunks: a view 2 bytes past a
    boundary is refused (NOT_HANDLED), not computed from shifted bytes."""
    n, k = 64, 512
    wb = np.ascontiguousarray(oracle.synthetic_weight(Q4_K, n, k, seed=11)).view(np.uint8).ravel()
    section = gpu.WeightsSection(np.concatenate([np.zeros(2, np.uint8), wb, np.zeros(256, np.uint8)]))
    W = section.view(2, wb.size, Q4_K, n, k)
    x = oracle.synthetic_acts(16, k, seed=3)
    try:
        with pytest.raises(gpu.NotHandled):
            tiled_b32(gpu, W, x)
    finally:
        W.release()
        section.free()
