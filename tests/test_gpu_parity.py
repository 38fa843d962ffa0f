"""Parity of the HIP path (libmimg.so, called through the C ABI) with the CPU
oracle on the same seeded inputs. The 8-bit block-256 products, the
activation quantizer and the decoder must be bit-exact; the float32-path
and block-32 kernels reproduce the reference's AVX2 lane order and are also
compared bit for bit with the oracle's restatement of it."""
import base64
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 64, 66, 67


def bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if a.shape != b.shape:
        return False
    same = a.view(np.uint32) == b.view(np.uint32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(same | both_nan))


def first_diff(a, b):
    a, b = np.asarray(a, np.float32).ravel(), np.asarray(b, np.float32).ravel()
    idx = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    if idx.size == 0:
        return "none"
    i = idx[0]
    return f"{idx.size} differ; first at {i}: {a[i]!r} vs {b[i]!r}"


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("dt,name", [(Q8_0, "q8_0"), (Q4_K, "q4_k"), (Q6_K, "q6_k")])
def test_dequantize_golden(gpu, dt, name):
    v = json.load(open(os.path.join(GOLDEN, "quant_golden.json")))[name]
    raw = base64.b64decode(v["bytes"])
    want = np.array(v["bits"], np.uint32)
    got = gpu.dequantize(dt, raw, want.size)
    assert np.array_equal(got.view(np.uint32), want)


@pytest.mark.parametrize("dt", [Q8_0, Q4_K, Q6_K])
def test_dequantize_random_bytes(gpu, oracle, dt):
    """Random block bytes (every scale pattern, including subnormal, inf and
    NaN f16 scales): GPU decode == oracle decode, bit for bit."""
    rng = np.random.default_rng(dt)
    nblk = 4096
    be, bb = oracle.BLOCK_ELEMS[dt], oracle.BLOCK_BYTES[dt]
    raw = rng.integers(0, 256, nblk * bb, dtype=np.uint8)
    got = gpu.dequantize(dt, raw, nblk * be)
    want = oracle.dequantize(dt, raw, nblk * be)
    assert bits_equal(got, want), first_diff(got, want)


def test_f16_scales_exhaustive(gpu, oracle):
    """Every f16 bit pattern as a Q8_0 scale with quant 1: d*1 on the GPU
    equals the oracle's exact conversion (subnormals included)."""
    h = np.arange(65536, dtype=np.uint16)
    raw = np.zeros((65536, 34), np.uint8)
    raw[:, 0] = h & 0xFF
    raw[:, 1] = h >> 8
    raw[:, 2] = 1
    got = gpu.dequantize(Q8_0, raw.ravel(), 65536 * 32).reshape(65536, 32)[:, 0]
    want = oracle.f16_to_f32(h)
    assert bits_equal(got, want), first_diff(got, want)


# ------------------------------------------------------------- encoders

@pytest.mark.parametrize("dt", [Q8_0, Q4_K, Q6_K])
def test_encoder_gpu_equals_oracle(gpu, oracle, dt):
    import hiprt

    rng = np.random.default_rng(21)
    n = 256 * 512
    x = rng.standard_normal(n).astype(np.float32) * np.float32(0.02)
    x[:256] *= 1000  # a block of larger values
    x[256:512] = 0  # an all-zero block
    nbytes = n // oracle.BLOCK_ELEMS[dt] * oracle.BLOCK_BYTES[dt]
    xd = hiprt.DeviceBuffer.from_array(x)
    out = hiprt.DeviceBuffer(nbytes)
    s = hiprt.Stream()
    gpu.quantize_dev(dt, xd.ptr, n, out.ptr, nbytes, s.handle)
    s.sync()
    assert np.array_equal(out.download(np.uint8), oracle.quantize(dt, x))


# ---------------------------------------------------- activation quantizer

@pytest.mark.parametrize("k", [2048, 4096, 4352, 14336])
@pytest.mark.parametrize("block", [256, 32])
def test_quantize_act_bitexact(gpu, oracle, block, k):
    """Rows of up to 16 chunks of 256 run in one workgroup, longer rows in
    several plus a scanning one: both, with refusals in the first and the
    last chunks."""
    import hiprt

    rows = 10
    rng = np.random.default_rng(block)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[1] *= np.float32(1e-30)
    x[2] *= np.float32(1e15)
    x[3, :256] = 0
    x[4, 100] = np.nan
    x[5, 1000] = np.float32(2.0 ** 61)
    # refusals in the row's last chunks (another workgroup than the first)
    x[7, k - 48] = np.nan
    x[8, k - 548] = -np.inf
    x[9, k - 1] = np.float32(2.0 ** 60)  # at the limit: not refused
    amax = np.abs(x[6, :block]).max()
    x[6, 1:5] = np.float32([0.5, 1.5, 2.5, -3.5]) * amax / np.float32(127)
    ws_bytes = gpu.a8_workspace_bytes(rows, k)
    off = gpu.a8_workspace_offsets(rows, k)
    ws = hiprt.DeviceBuffer(ws_bytes)
    ws.zero()
    xd = hiprt.DeviceBuffer.from_array(x)
    s = hiprt.Stream()
    gpu.quantize_act_dev(xd.ptr, rows, k, block, ws.ptr, ws_bytes, s.handle)
    s.sync()
    h = ws.download(np.uint8)
    q = h[off[0]:off[0] + rows * k].view(np.int8).reshape(rows, k)
    d = h[off[1]:off[1] + rows * k // 32 * 4].view(np.float32).reshape(rows, -1)
    xs = h[off[2]:off[2] + rows * k // 32 * 2].view(np.int16).reshape(rows, -1)
    ys = h[off[3]:off[3] + rows * k // 16 * 2].view(np.int16).reshape(rows, -1)
    dbs = h[off[4]:off[4] + rows * k // 32 * 4].view(np.float32).reshape(rows, -1)
    ok = h[off[5]:off[5] + rows * 4].view(np.int32)
    for i in range(rows):
        a = oracle.Act(x[i], block)
        assert bool(ok[i]) == a.ok, i
        if not a.ok:
            continue
        assert np.array_equal(q[i], a.q), i
        assert bits_equal(d[i], a.d), i
        assert np.array_equal(xs[i], a.xs), i
        assert bits_equal(dbs[i], a.dbs), i
        assert np.array_equal(ys[i], a.q.astype(np.int32).reshape(-1, 16).sum(1)), i


@pytest.mark.parametrize("block", [256, 32])
def test_quantize_act_many_long_rows(gpu, oracle, block):
    """64 rows of K = 14336 (one workgroup a row from 64 rows): every row
    bit for bit the restatement, refusals anywhere in the row."""
    import hiprt

    rows, k = 64, 14336
    rng = np.random.default_rng(64 + block)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[3, 14000] = np.nan
    x[17, 9000] = np.float32(2.0 ** 61)
    x[40, 255] = -np.inf
    x[63, 14335] = np.float32(2.0 ** 60)  # at the limit: not refused
    ws_bytes = gpu.a8_workspace_bytes(rows, k)
    off = gpu.a8_workspace_offsets(rows, k)
    ws = hiprt.DeviceBuffer(ws_bytes)
    ws.zero()
    xd = hiprt.DeviceBuffer.from_array(x)
    s = hiprt.Stream()
    gpu.quantize_act_dev(xd.ptr, rows, k, block, ws.ptr, ws_bytes, s.handle)
    s.sync()
    h = ws.download(np.uint8)
    q = h[off[0]:off[0] + rows * k].view(np.int8).reshape(rows, k)
    d = h[off[1]:off[1] + rows * k // 32 * 4].view(np.float32).reshape(rows, -1)
    xs = h[off[2]:off[2] + rows * k // 32 * 2].view(np.int16).reshape(rows, -1)
    ok = h[off[5]:off[5] + rows * 4].view(np.int32)
    for i in range(rows):
        a = oracle.Act(x[i], block)
        assert bool(ok[i]) == a.ok, i
        if not a.ok:
            continue
        assert np.array_equal(q[i], a.q), i
        assert bits_equal(d[i], a.d), i
        assert np.array_equal(xs[i], a.xs), i


# ------------------------------------------- block-256 8-bit products (GEMV)

def _weights(oracle, dt, n, k, seed):
    return oracle.synthetic_weight(dt, n, k, seed)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("n,k", [(1, 256), (33, 2048), (200, 5632), (64, 14336), (4096, 512)])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
def test_linear_a8k_bitexact(gpu, oracle, dt, n, k, rows):
    wb = _weights(oracle, dt, n, k, seed=n + k)
    x = oracle.synthetic_acts(rows, k, seed=rows)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows", [5, 6, 7, 9, 17])
def test_linear_a8k_row_counts(gpu, oracle, dt, rows):
    """Odd row counts and more than 8 rows (several launches) give the same
    bits as the reference, which computes rows independently
    (TestDequantMatmulA8RowsTogether, interp/transformer_test.go:303-349)."""
    n, k = 96, 1024
    wb = _weights(oracle, dt, n, k, seed=3)
    x = oracle.synthetic_acts(rows, k, seed=rows + 100)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
    assert bits_equal(got, want), first_diff(got, want)
    one = np.stack([gpu.dequant_matmul_a8(W, x[i:i + 1], block=256)[0] for i in range(rows)])
    assert bits_equal(got, one)
    W.release()


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
def test_linear_a8k_special_inputs(gpu, oracle, dt):
    """The inputs of TestDotQ8KReference (reference q8k_test.go:104-187):
    tiny and huge activations, a zero block, the largest finite f16 scales
    with all-ones quants, subnormal f16 scales."""
    from test_oracle import _special_rows

    k = 5632
    rng = np.random.default_rng(14)
    x = rng.standard_normal((5, k)).astype(np.float32)
    x[1] *= np.float32(1e-30)
    x[2] *= np.float32(1e15)
    x[3, :256] = 0
    rows = [_special_rows(dt, k, t, rng, oracle) for t in range(3)]
    wb = np.frombuffer(b"".join(rows), np.uint8)
    W = gpu.Weight(wb, dt, 3, k)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, 3, k, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,n,k", [(16, 64, 256), (64, 100, 1024), (130, 300, 4096), (257, 129, 2048),
                                      (128, 1024, 14336)])
def test_gemm_a8k_bitexact(gpu, oracle, dt, rows, n, k):
    """Prefill sizes (16 rows and more) run on the int8 MFMA GEMM: ragged
    row and column counts, one and several 64x128 tiles, K from one block
    to 56; bit for bit the reference, whose tile kernels equal its one-row
    kernel (reference amx_test.go:41-141)."""
    wb = _weights(oracle, dt, n, k, seed=rows + n)
    x = oracle.synthetic_acts(rows, k, seed=rows + 1)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt,rows,n,k", [(Q4_K, 1100, 4100, 256), (Q6_K, 1000, 4160, 1024), (Q4_K, 2050, 2070, 2048),
                                         (Q6_K, 1290, 3000, 768), (Q6_K, 1030, 4096, 2304)])
def test_gemm_a8k_wide_tiles_bitexact(gpu, oracle, dt, rows, n, k):
    """Grids of at least 256 tiles of 128 x 128 run on the 32x32x32 kernel
    (ping-pong waves): ragged last weight and activation tiles, K from one
    block up, Q6_K rows whose blocks sit at every offset mod 16; bit for bit
    the reference."""
    wb = _weights(oracle, dt, n, k, seed=rows + n + k)
    x = oracle.synthetic_acts(rows, k, seed=rows + 2)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=16)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
def test_gemm_a8k_wide_tiles_refusals_and_bias(gpu, oracle, dt):
    """The 32x32x32 kernel's refused pairs (a NaN activation row, a row
    above 2^60, weight rows with an infinite or NaN block scale) take the
    float32 path, and bias is added as s + bias[j]."""
    n, k, rows = 4100, 512, 1040
    wb = bytearray(_weights(oracle, dt, n, k, seed=18).tobytes())
    rb = len(wb) // n
    f = 208 if dt == Q6_K else 2
    for j, blk in ((5, 0), (3000, 1)):
        o = rb * j + blk * (210 if dt == Q6_K else 144) + f
        wb[o:o + 2] = b"\x00\x7c" if j == 5 else b"\x01\x7e"
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=19)
    x[7, 3] = np.nan
    x[900, 100] = np.float32(1e30)
    bias = np.random.default_rng(20).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256, threads=16)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,k", [(1, 1024), (3, 1024), (12, 1024), (40, 1024), (6, 1024), (8, 4096), (7, 14336)])
def test_linear_a8k_refusals_and_bias(gpu, oracle, dt, rows, k):
    """Rows of x with NaN/Inf/huge values and rows of w with a non-finite
    block scale take the float32 path (reference interp/fast.go:323-377);
    bias is added as s + bias[j]. 6..8 rows run on the matrix-core GEMV,
    with 4 waves per workgroup (K = 1024) and, for Q6_K, 12 (three
    workgroups)."""
    n = 40
    wb = bytearray(_weights(oracle, dt, n, k, seed=8).tobytes())
    rb = len(wb) // n
    f = 208 if dt == Q6_K else 2  # Q4_K: dmin
    for j, blk in ((5, 0), (17, 3)):
        o = rb * j + blk * (210 if dt == Q6_K else 144) + f
        wb[o:o + 2] = b"\x00\x7c" if j == 5 else b"\x01\x7e"  # +inf, NaN
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=9)
    x[0, 3] = np.nan
    if rows > 2:
        x[2, 700] = np.float32(1e30)
    bias = np.random.default_rng(10).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    assert W.info()[1] == 2
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


def test_linear_a8k_llama_blocks(gpu, oracle):
    """Weights written by llama.cpp's quantizer (reference testdata/llama)."""
    z = np.load(os.path.join(GOLDEN, "llama_tensors.npz"))
    for name in ("blk_0_attn_q_weight", "blk_0_ffn_down_weight", "output_weight", "token_embd_weight"):
        raw, shape, dt = z[name + "__bytes"], z[name + "__shape"], int(z[name + "__dtype"][0])
        n, k = int(shape[0]), int(shape[1])
        x = oracle.synthetic_acts(3, k, seed=11)
        W = gpu.Weight(raw, dt, n, k)
        got = gpu.dequant_matmul_a8(W, x, block=256)
        want = oracle.linear_a8(x, raw, dt, n, k, block=256)
        W.release()
        assert bits_equal(got, want), (name, first_diff(got, want))


# ------------------------------------------- device entry points and groups

def _dev_linear(gpu, weights, x, biases=None, group=True, prequant=False):
    """Runs weights on x through the device entry points; returns [y_i]."""
    import hiprt

    rows, k = x.shape
    xd = hiprt.DeviceBuffer.from_array(x)
    ws_bytes = gpu.a8_workspace_bytes(rows, k)
    ws = hiprt.DeviceBuffer(ws_bytes)
    ys = [hiprt.DeviceBuffer(rows * w.n * 4) for w in weights]
    bds = [None if b is None else hiprt.DeviceBuffer.from_array(b) for b in (biases or [None] * len(weights))]
    s = hiprt.Stream()
    if prequant:
        gpu.quantize_act_dev(xd.ptr, rows, k, 256, ws.ptr, ws_bytes, s.handle)
        for w, y, b in zip(weights, ys, bds):
            gpu.matmul_a8_quantized_dev(w, xd.ptr, rows, b.ptr if b else None, 256, y.ptr, ws.ptr, ws_bytes, s.handle)
    elif group:
        gpu.linear_a8_group_dev(weights, xd.ptr, rows, [b.ptr if b else 0 for b in bds], 256,
                                [y.ptr for y in ys], ws.ptr, ws_bytes, s.handle)
    else:
        for w, y, b in zip(weights, ys, bds):
            gpu.linear_a8_dev(w, xd.ptr, rows, b.ptr if b else None, 256, y.ptr, ws.ptr, ws_bytes, s.handle)
    s.sync()
    return [y.download(np.float32).reshape(rows, w.n) for y, w in zip(ys, weights)]


@pytest.mark.parametrize("shape", ["small", "llama8b"])
@pytest.mark.parametrize("rows", [1, 3, 8])
def test_group_qkv_bitexact(gpu, oracle, rows, shape):
    """q, k (Q4_K) and v (Q6_K) sharing one input in one grouped call (a single
    fused launch at one row; at the Llama-3-8B shape its 768 tiles run three
    to a workgroup) equal the separate reference products."""
    k = 4096
    nq, nkv = (512, 128) if shape == "small" else (4096, 1024)
    specs = [(Q4_K, nq, 21), (Q4_K, nkv, 22), (Q6_K, nkv, 23)]
    wbs = [_weights(oracle, dt, n, k, seed) for dt, n, seed in specs]
    W = [gpu.Weight(wb, dt, n, k) for wb, (dt, n, _) in zip(wbs, specs)]
    x = oracle.synthetic_acts(rows, k, seed=24)
    bias = [np.random.default_rng(i).standard_normal(n).astype(np.float32) for i, (_, n, _) in enumerate(specs)]
    got = _dev_linear(gpu, W, x, biases=[bias[0], None, bias[2]])
    for i, ((dt, n, _), wb) in enumerate(zip(specs, wbs)):
        want = oracle.linear_a8(x, wb, dt, n, k, bias=bias[i] if i != 1 else None, block=256)
        assert bits_equal(got[i], want), (i, first_diff(got[i], want))
    for w in W:
        w.release()


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("n,k", [(300, 14336), (4100, 4096), (7, 256)])
def test_pairs_kernel_one_row_bitexact(gpu, oracle, dt, n, k):
    """The pre-quantized path (quantize launch + pair kernel) at one row."""
    wb = _weights(oracle, dt, n, k, seed=31)
    W = gpu.Weight(wb, dt, n, k)
    x = oracle.synthetic_acts(1, k, seed=32)
    got = _dev_linear(gpu, [W], x, prequant=True)[0]
    want = oracle.linear_a8(x, wb, dt, n, k, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("n,k", [(4096, 14336), (4099, 4096), (1, 2048), (1025, 6144), (3, 16384)])
def test_q6k_one_row_gemv_bitexact(gpu, oracle, n, k):
    """Q6_K at one activation row (the pair kernel on pre-quantized
    activations): ragged last tiles of rows, odd row counts, K from 8 to 64
    blocks; bit for bit the reference."""
    wb = _weights(oracle, Q6_K, n, k, seed=n + 5)
    W = gpu.Weight(wb, Q6_K, n, k)
    x = oracle.synthetic_acts(1, k, seed=k + 5)
    got = _dev_linear(gpu, [W], x, prequant=True)[0]
    want = oracle.linear_a8(x, wb, Q6_K, n, k, block=256, threads=16)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


def test_q6k_one_row_gemv_refusals_bias_and_group(gpu, oracle):
    """The one-row Q6_K GEMV with a weight row whose block scale is infinite
    (float32 path), bias, two matrices in one launch, then a refused
    activation row (every row on the float32 path)."""
    k = 4096
    wbs = []
    for n, seed in ((700, 41), (300, 42)):
        wb = bytearray(_weights(oracle, Q6_K, n, k, seed=seed).tobytes())
        rb = len(wb) // n
        o = rb * 17 + 5 * 210 + 208
        wb[o:o + 2] = b"\x00\x7c"
        wbs.append(np.frombuffer(bytes(wb), np.uint8))
    W = [gpu.Weight(wb, Q6_K, wb.size // (k // 256 * 210), k) for wb in wbs]
    biases = [np.random.default_rng(i).standard_normal(w.n).astype(np.float32) for i, w in enumerate(W)]
    x = oracle.synthetic_acts(1, k, seed=43)
    import hiprt

    for case in range(2):
        if case == 1:
            x[0, 2000] = np.nan
        xd = hiprt.DeviceBuffer.from_array(x)
        wsb = gpu.a8_workspace_bytes(1, k)
        ws = hiprt.DeviceBuffer(wsb)
        ys = [hiprt.DeviceBuffer(w.n * 4) for w in W]
        bds = [hiprt.DeviceBuffer.from_array(b) for b in biases]
        st = hiprt.Stream()
        gpu.quantize_act_dev(xd.ptr, 1, k, 256, ws.ptr, wsb, st.handle)
        gpu.matmul_a8_quantized_group_dev(W, xd.ptr, 1, [b.ptr for b in bds], 256, [y.ptr for y in ys], ws.ptr, wsb,
                                          st.handle)
        st.sync()
        got = [y.download(np.float32).reshape(1, w.n) for y, w in zip(ys, W)]
        for i, (w, wb) in enumerate(zip(W, wbs)):
            want = oracle.linear_a8(x, wb, Q6_K, w.n, k, bias=biases[i], block=256)
            assert bits_equal(got[i], want), (case, i, first_diff(got[i], want))
    for w in W:
        w.release()


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("n,k", [(300, 14336), (4100, 4096), (8200, 2048), (7, 256), (33, 768)])
@pytest.mark.parametrize("rows", [4, 5, 8])
def test_mfma_gemv_bitexact(gpu, oracle, dt, n, k, rows):
    """4..8 activation rows run on the int8 matrix-core GEMV: ragged last
    tile of 16 rows, K from one block to 56, workgroups of 4 waves (Q4_K;
    Q6_K with K of 1 and 3 blocks: idle and uneven waves), Q6_K 8 waves
    (513 tiles of 8 blocks) and 12 (19 and 257 tiles: 56 and 16 blocks
    split unevenly), odd block counts (Q6_K rows 2-byte aligned); the same
    bits as the reference's per-row products."""
    wb = _weights(oracle, dt, n, k, seed=n + rows)
    W = gpu.Weight(wb, dt, n, k)
    x = oracle.synthetic_acts(rows, k, seed=rows + 7)
    got = _dev_linear(gpu, [W], x, prequant=True)[0]
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


def test_output_overlapping_input_refused(gpu, oracle):
    """Every workgroup reads all of x while others write y, so an output
    that overlaps the input is an argument error (before any launch), for
    the one-row fused launch, the pre-quantized products and the groups."""
    import hiprt

    k, n = 1024, 64
    W = gpu.Weight(_weights(oracle, Q4_K, n, k, seed=5), Q4_K, n, k)
    buf = hiprt.DeviceBuffer(8 * k * 4)
    wsb = gpu.a8_workspace_bytes(8, k)
    ws = hiprt.DeviceBuffer(wsb)
    s = hiprt.Stream()
    for rows in (1, 8):
        with pytest.raises(gpu.MimgError) as e:
            gpu.linear_a8_group_dev([W], buf.ptr, rows, None, 256, [buf.ptr + 256], ws.ptr, wsb, s.handle)
        assert not isinstance(e.value, gpu.NotHandled)
        with pytest.raises(gpu.MimgError):
            gpu.matmul_a8_quantized_dev(W, buf.ptr, rows, None, 256, buf.ptr, ws.ptr, wsb, s.handle)
        with pytest.raises(gpu.MimgError):
            gpu.matmul_a8_quantized_group_dev([W], buf.ptr, rows, None, 256, [buf.ptr], ws.ptr, wsb, s.handle)
        with pytest.raises(gpu.MimgError):
            gpu.linear_f32_dev(W, buf.ptr, rows, None, buf.ptr + 1024, s.handle)
        with pytest.raises(gpu.MimgError):
            gpu.linear_f32_mfma_dev(W, buf.ptr, rows, None, buf.ptr, s.handle)
    # the fused norm GEMV: y[i] against x, resid, scale and x_out
    other = hiprt.DeviceBuffer(4 * k * 4)
    x, resid, scale, x_out = (other.ptr + i * k * 4 for i in range(4))
    for y in (x, resid, scale, x_out, x + 64):
        with pytest.raises(gpu.MimgError) as e:
            gpu.rms_norm_linear_a8_group_dev([W], x, resid, scale, 1e-5, x_out, None, [y], s.handle)
        assert not isinstance(e.value, gpu.NotHandled)
    own = hiprt.DeviceBuffer(n * 4)
    gpu.rms_norm_linear_a8_group_dev([W], x, resid, scale, 1e-5, x_out, None, [own.ptr], s.handle)
    s.sync()
    W.release()


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
def test_fused_refusals_large_k(gpu, oracle, dt):
    """The fused one-row kernel at K = 14336 with a refused weight row, then
    with a refused activation row (all products on the float32 path)."""
    n, k = 96, 14336
    wb = bytearray(_weights(oracle, dt, n, k, seed=33).tobytes())
    rb = len(wb) // n
    o = rb * 40 + 3 * (210 if dt == Q6_K else 144) + (208 if dt == Q6_K else 0)
    wb[o:o + 2] = b"\x00\xfc"  # -inf
    wb = np.frombuffer(bytes(wb), np.uint8)
    W = gpu.Weight(wb, dt, n, k)
    bias = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    x = oracle.synthetic_acts(1, k, seed=34)
    got = _dev_linear(gpu, [W], x, biases=[bias], group=False)[0]
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256)
    assert bits_equal(got, want), first_diff(got, want)
    x[0, 9999] = np.float32(3e19)  # above 2^60: the row is refused
    got = _dev_linear(gpu, [W], x, biases=[bias], group=False)[0]
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
def test_fused_teams_refusals(gpu, oracle, dt):
    """The one-row fused launch with two tiles of 8 rows per workgroup (a
    4096 x 4096 matrix: 512 tiles, the second team's rows 8..15 in the
    first workgroup) with a refused weight row in that team's tile, then a
    refused activation row (every product on the float32 path)."""
    n, k = 4096, 4096
    bb = 210 if dt == Q6_K else 144
    wb = bytearray(_weights(oracle, dt, n, k, seed=37).tobytes())
    rb = len(wb) // n
    for row in (9, 4000):
        o = rb * row + 2 * bb + (208 if dt == Q6_K else 0)
        wb[o:o + 2] = b"\x00\x7c"  # +inf block scale
    wb = np.frombuffer(bytes(wb), np.uint8)
    W = gpu.Weight(wb, dt, n, k)
    assert W.info()[1] == 2
    bias = np.random.default_rng(6).standard_normal(n).astype(np.float32)
    x = oracle.synthetic_acts(1, k, seed=38)
    for case in range(2):
        if case == 1:
            x[0, 3333] = np.nan  # the row is refused
        got = _dev_linear(gpu, [W], x, biases=[bias], group=False)[0]
        want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256)
        assert bits_equal(got, want), (case, first_diff(got, want))
    W.release()


@pytest.mark.parametrize("k,n", [(1024, 64), (4096, 4096)])
def test_fused_quantizer_ties(gpu, oracle, k, n):
    """Activations on exact half-integer steps (127 x / amax = n + 1/2) and
    next to them: the in-kernel quantizer must round exactly as the reference
    (one team a workgroup, 16 threads a block; 4096 x 4096: two teams, 32
    threads a block)."""
    wb = _weights(oracle, Q4_K, n, k, seed=35)
    W = gpu.Weight(wb, Q4_K, n, k)
    rng = np.random.default_rng(36)
    x = rng.standard_normal((1, k)).astype(np.float32)
    for b in range(k // 256):
        amax = np.float32(127 * 2.0 ** rng.integers(-3, 4))  # amax/127 a power of two: exact ties exist
        blk = x[0, 256 * b:256 * b + 256]
        blk[:] = np.clip(blk, -amax, amax)
        blk[0] = amax
        step = amax / np.float32(127)
        for i, h in enumerate(np.arange(-20.5, 21.5, 1.0)):
            blk[1 + i] = np.float32(h) * step
            blk[100 + i] = np.nextafter(np.float32(h) * step, np.float32(np.inf))
            blk[150 + i] = np.nextafter(np.float32(h) * step, np.float32(-np.inf))
    got = _dev_linear(gpu, [W], x, group=False)[0]
    want = oracle.linear_a8(x, wb, Q4_K, n, k, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


# ----------------------------------------------- Q8_0 x blocks of 32 (a8.v1)

@pytest.mark.parametrize("rows", [1, 4, 8, 11])
def test_linear_q8_0_a8_bitexact(gpu, oracle, rows):
    n, k = 150, 4096 + 32
    wb = _weights(oracle, Q8_0, n, k, seed=12)
    x = oracle.synthetic_acts(rows, k, seed=13)
    x[0, 40] = np.inf
    bias = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, Q8_0, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=32)
    want = oracle.linear_a8(x, wb, Q8_0, n, k, bias=bias, block=32)
    # Q8_0 with blocks of 256 has no 8-bit kernel: the float32 path
    got256 = gpu.dequant_matmul_a8(W, x, block=256)
    want256 = oracle.linear_a8(x, wb, Q8_0, n, k, block=256)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)
    assert bits_equal(got256, want256), first_diff(got256, want256)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows", [1, 3, 8, 11])
def test_linear_kquant_a8_block32_bitexact(gpu, oracle, dt, rows):
    """Q4_K/Q6_K with activation blocks of 32 (dequant_matmul_a8.v1): the
    lane order of dotQ4KQ8AVX2/dotQ6KQ8AVX2 as the oracle restates it, bit
    for bit, with a refused activation row (float32 path), a weight row with
    a non-finite scale, bias, and more than 8 rows (DotF32 fallback order)."""
    n, k = 70, 2048
    wb = bytearray(_weights(oracle, dt, n, k, seed=21).tobytes())
    rb = len(wb) // n
    o = rb * 9 + (208 if dt == Q6_K else 0)
    wb[o:o + 2] = b"\x00\x7c"  # row 9: +inf block scale
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=22)
    x[rows - 1, 7] = np.nan
    bias = np.random.default_rng(23).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=32)
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=32)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


# ------------------------------------------------- float32-activation path

@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("rows", [1, 8, 9])
def test_linear_f32_bitexact(gpu, oracle, dt, rows):
    """dequant_matmul.v1: the fused order for <= 8 rows, decode-then-DotF32
    for more (reference kernels.go:122-204)."""
    n, k = 70, 1024
    wb = _weights(oracle, dt, n, k, seed=14)
    x = oracle.synthetic_acts(rows, k, seed=15)
    bias = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul(W, x, bias=bias)
    want = oracle.linear_f32(x, wb, dt, n, k, bias=bias)
    W.release()
    assert bits_equal(got, want), first_diff(got, want)


# ------------------------------------------------------------ errors

def test_errors_are_reported_not_fatal(gpu, oracle):
    wb = _weights(oracle, Q4_K, 4, 256, seed=1)
    with pytest.raises(gpu.MimgError):
        gpu.Weight(wb[:-1], Q4_K, 4, 256)  # wrong byte count
    W = gpu.Weight(wb, Q4_K, 4, 256)
    with pytest.raises(gpu.MimgError):
        gpu.dequant_matmul_a8(W, np.zeros((1, 256), np.float32), block=64)  # block must be 32 or 256
    # the same bytes register once
    W2 = gpu.Weight(wb, Q4_K, 4, 256)
    assert W2.handle == W.handle
    W.release()


# --------------------------------------------------- full-size shapes (cfg0/1)

CFG1 = [  # (name, N, K, dtype, seed): Llama-3-8B layer, M = 1
    ("q", 4096, 4096, Q4_K, 0), ("k", 1024, 4096, Q4_K, 1), ("v", 1024, 4096, Q6_K, 2),
    ("o", 4096, 4096, Q4_K, 3), ("gate", 14336, 4096, Q4_K, 4), ("up", 14336, 4096, Q4_K, 5),
    ("down", 4096, 14336, Q6_K, 6),
]


@pytest.mark.parametrize("name,n,k,dt,seed", CFG1)
def test_cfg1_layer_shapes_bitexact(gpu, oracle, name, n, k, dt, seed):
    """The BASELINE layer shapes at full size, M = 1 and M = 8: bit-exact."""
    wb = _weights(oracle, dt, n, k, seed)
    W = gpu.Weight(wb, dt, n, k)
    for rows in (1, 8):
        x = oracle.synthetic_acts(rows, k, seed=1)
        got = gpu.dequant_matmul_a8(W, x, block=256)
        want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
        assert bits_equal(got, want), (name, rows, first_diff(got, want))
    W.release()


# ------------------------------------------------------ weight registration

def test_register_same_bytes_shares_and_other_bytes_upload(gpu, oracle):
    """The same (address, length, dtype, shape) returns the same handle with
    one more reference; other bytes written at that address (a file closed
    and another mapped there) are uploaded afresh, and the old handle keeps
    computing with its own copy until released."""
    import ctypes

    lib = gpu.load()
    n, k = 64, 512
    buf = np.ascontiguousarray(oracle.synthetic_weight(Q4_K, n, k, seed=31))
    first = buf.copy()
    x = oracle.synthetic_acts(1, k, seed=32)

    def reg():
        h = ctypes.c_uint64()
        assert lib.mimg_register_weight(buf.ctypes.data, buf.size, Q4_K, n, k, ctypes.byref(h)) == 0
        return h.value

    def run(h):
        y = np.empty((1, n), np.float32)
        assert lib.mimg_dequant_matmul_a8(h, x.ctypes.data, 1, None, 256, y.ctypes.data) == 0
        return y

    h1 = reg()
    assert reg() == h1                      # second reference, no upload
    assert lib.mimg_release_weight(h1) == 0  # drops one: still valid
    assert bits_equal(run(h1), oracle.linear_a8(x, first, Q4_K, n, k, block=256))
    buf[:] = oracle.synthetic_weight(Q4_K, n, k, seed=33)  # new bytes, same address
    h2 = reg()
    assert h2 != h1
    assert bits_equal(run(h2), oracle.linear_a8(x, buf, Q4_K, n, k, block=256))
    assert bits_equal(run(h1), oracle.linear_a8(x, first, Q4_K, n, k, block=256))
    assert lib.mimg_release_weight(h1) == 0
    assert lib.mimg_release_weight(h1) < 0   # gone
    assert lib.mimg_release_weight(h2) == 0
