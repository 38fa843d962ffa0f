"""BASELINE configs 0 and 2 at their full shapes, on the GPU through the C
ABI, against the CPU oracle on the same bytes.

cfg0 is the single 4096 x 4096 Q4_K product of one activation row (W from
seed 0, x from seed 1), as dequant_matmul_a8.v2 with blocks of 256 and as
dequant_matmul.v1. cfg2 is the prefill: the gate (14336 x 4096 Q4_K) and
down (4096 x 14336 Q6_K) products at 64, 512 and 2048 activation rows, which
run on the int8 matrix-core GEMM. The reference's tile kernels give the
bits of its one-row kernel (reference internal/kernels/amx_test.go:41-141,
interp/transformer_test.go:297-349), so every output is compared bit for
bit with the oracle's dotQ8KRef restatement (q8k_test.go:38-102)."""
import functools

import numpy as np
import pytest

from test_gpu_parity import bits_equal, first_diff

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 64, 66, 67


@functools.lru_cache(maxsize=4)
def _weight_bytes(dt, n, k, seed):
    import mimref

    return mimref.synthetic_weight(dt, n, k, seed)


@pytest.fixture(scope="module")
def layer_weights(gpu):
    made = {}

    def get(dt, n, k, seed):
        key = (dt, n, k, seed)
        if key not in made:
            wb = _weight_bytes(dt, n, k, seed)
            made[key] = (wb, gpu.Weight(wb, dt, n, k))
        return made[key]

    yield get
    for _, w in made.values():
        w.release()


def test_cfg0_q4k_matvec(gpu, oracle, layer_weights):
    """cfg0: y = W x for W 4096 x 4096 Q4_K (seed 0), x f32[4096] (seed 1):
    the 8-bit path bit-exact with dotQ8KRef, the float32 path bit-exact with
    the oracle's restatement of dotQ4KAVX2's lane order."""
    n = k = 4096
    wb, W = layer_weights(Q4_K, n, k, 0)
    x = oracle.synthetic_acts(1, k, seed=1)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, Q4_K, n, k, block=256, threads=16)
    assert bits_equal(got, want), first_diff(got, want)
    got = gpu.dequant_matmul(W, x)
    want = oracle.linear_f32(x, wb, Q4_K, n, k, threads=16)
    assert bits_equal(got, want), first_diff(got, want)


CFG2 = [("gate", 14336, 4096, Q4_K, 4), ("down", 4096, 14336, Q6_K, 6)]


@pytest.mark.parametrize("rows", [64, 512, 2048])
@pytest.mark.parametrize("name,n,k,dt,seed", CFG2, ids=[c[0] for c in CFG2])
def test_cfg2_prefill_layer_shapes_bitexact(gpu, oracle, layer_weights, name, n, k, dt, seed, rows):
    """cfg2 block-256 prefill at the layer shapes: every one of the rows x N
    outputs equal to the oracle's, bit for bit."""
    wb, W = layer_weights(dt, n, k, seed)
    x = oracle.synthetic_acts(rows, k, seed=100 + rows)
    print(f"cfg2 {name} rows {rows}", flush=True)
    got = gpu.dequant_matmul_a8(W, x, block=256)
    want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=16)
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K], ids=["q4_k", "q6_k"])
@pytest.mark.parametrize("rows,n,k", [(16, 100, 256), (33, 4096, 1024), (64, 1000, 2048), (50, 24, 512)])
def test_small_grid_prefill_bitexact_with_refusals(gpu, oracle, dt, rows, n, k):
    """16..64 activation rows on few weight rows (the k-step-split kernel:
    16 weight rows a workgroup, the four waves on the four k steps of each
    block): partial tiles of weight and activation rows, a refused
    activation row (NaN) and a weight row with an infinite block scale; every
    output equal to the oracle's, bit for bit."""
    bb, doff = (144, 0) if dt == Q4_K else (210, 208)
    wb = bytearray(oracle.synthetic_weight(dt, n, k, seed=rows + n).tobytes())
    rb = len(wb) // n
    bad = min(7, n - 1)
    wb[rb * bad + bb * (k // 256 - 1) + doff:rb * bad + bb * (k // 256 - 1) + doff + 2] = b"\x00\x7c"
    wb = np.frombuffer(bytes(wb), np.uint8)
    x = oracle.synthetic_acts(rows, k, seed=rows)
    x[rows // 2, 3] = np.nan
    bias = np.random.default_rng(rows).standard_normal(n).astype(np.float32)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=256)
    W.release()
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256, threads=16)
    assert bits_equal(got, want), first_diff(got, want)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K], ids=["q4_k", "q6_k"])
@pytest.mark.parametrize("rows,n,k", [(512, 1024, 4096), (130, 1024, 4096), (300, 520, 2048), (1000, 2000, 1024)])
def test_few_weight_rows_many_activation_rows_bitexact(gpu, oracle, dt, rows, n, k):
    """More than 64 activation rows on few weight rows (a prompt's k and v
    products: 1024 x 4096 at 512 rows), where the 128 x 128 tiles leave CUs
    idle and a small-grid tiling runs: partial tiles, a refused activation
    row (NaN) and bias; every output equal to the oracle's, bit for bit."""
    wb = oracle.synthetic_weight(dt, n, k, seed=rows + n + k)
    x = oracle.synthetic_acts(rows, k, seed=rows + 1)
    x[rows // 3, 5] = np.nan
    bias = np.random.default_rng(rows + 2).standard_normal(n).astype(np.float32)
    print(f"few weight rows: dt {dt} rows {rows} n {n} k {k}", flush=True)
    W = gpu.Weight(wb, dt, n, k)
    got = gpu.dequant_matmul_a8(W, x, bias=bias, block=256)
    W.release()
    want = oracle.linear_a8(x, wb, dt, n, k, bias=bias, block=256, threads=16)
    assert bits_equal(got, want), first_diff(got, want)
