"""Checks of the C restatement of the decoder ops (oracle/mimref.c:
mref_expsum_f32, mref_scores, mref_attend_row/mref_attention,
mref_silu_mul) that do not retype its formulas: float64 brute force within
error bounds that a dropped term, a wrong index or a transposed operand
would exceed, closed forms (exp(0) = 1, the clamp to 0 below the smallest
normal result), the identities the reference states (ScoresF16 equals
ScoresF32 on the converted keys; the weighted sum equals row-by-row axpy
with fma), and the piece split of the reference's parallel(). The AVX2 lane
orders themselves are restated from attn_amd64.s; no golden output of
those kernels exists (the reference cannot run here), so their bits are
pinned only through the reference fixtures' tolerances
(tests/test_decoder_oracle.py)."""
import math

import numpy as np
import pytest

ULP = 2.0 ** -23


def test_exp_closed_forms(oracle):
    x, s = oracle.expsum_f32(np.zeros(16, np.float32), 0.0)
    assert np.all(x == 1.0) and s == 16.0
    # below the limit of normal results (and -inf): exactly 0
    x, s = oracle.expsum_f32(np.array([-88.0, -1e30, -np.inf, -87.0] * 2, np.float32), 0.0)
    assert x[0] == 0 and x[1] == 0 and x[2] == 0 and x[3] > 0


def test_exp_accuracy_against_float64(oracle):
    """Cephes' expf is within a few ulp of exp over [-87, 0]; a wrong
    polynomial coefficient or a dropped ln2 part is far outside this."""
    t = np.linspace(-87.0, 0.0, 200001).astype(np.float32)
    x, _ = oracle.expsum_f32(t, 0.0)
    want = np.exp(t.astype(np.float64))
    rel = np.abs(x.astype(np.float64) - want) / want
    assert np.max(rel) <= 2.5 * ULP, np.max(rel)


@pytest.mark.parametrize("n", [1, 7, 8, 9, 16, 23, 100])
def test_expsum_sum_and_tail(oracle, n):
    """The sum is the exponentials' sum within n ulp; the tail (past
    n&~7) is f32(exp(f64)) exactly."""
    rng = np.random.default_rng(n)
    v = (rng.standard_normal(n) * 3).astype(np.float32)
    m = np.float32(v.max())
    x, s = oracle.expsum_f32(v, m)
    nv = n & ~7 if n >= 8 else 0
    tail = np.exp((v[nv:] - m).astype(np.float64)).astype(np.float32)
    assert np.array_equal(x[nv:], tail)
    assert abs(float(s) - float(np.sum(x.astype(np.float64)))) <= n * ULP * float(s)


@pytest.mark.parametrize("n,d", [(1, 8), (4, 64), (5, 64), (7, 128), (13, 32)])
def test_scores_against_float64(oracle, n, d):
    rng = np.random.default_rng(n * d)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal((n, d)).astype(np.float32)
    scale = np.float32(1.0 / math.sqrt(d))
    got = oracle.scores(q, k, scale)
    exact = (k.astype(np.float64) @ q.astype(np.float64)) * float(scale)
    bound = (d + 2) * ULP * (np.abs(k.astype(np.float64)) @ np.abs(q.astype(np.float64))) * float(scale)
    assert np.all(np.abs(got - exact) <= bound)
    # keys stored as f16 give the scores of the converted keys, bit for bit
    k16 = k.astype(np.float16)
    assert np.array_equal(oracle.scores(q, k16, scale).view(np.uint32),
                          oracle.scores(q, k16.astype(np.float32), scale).view(np.uint32))


@pytest.mark.parametrize("n,d", [(1, 64), (3, 64), (8, 64), (37, 128), (300, 64)])
def test_attention_against_float64(oracle, n, d):
    """Softmax attention of one query within a few ulp of the float64
    result; a missing scale, a wrong max or an off-by-one range fails."""
    rng = np.random.default_rng(n + d)
    q = rng.standard_normal((1, 1, d)).astype(np.float32)
    kc = rng.standard_normal((1, n + 5, d)).astype(np.float32)
    vc = rng.standard_normal((1, n + 5, d)).astype(np.float32)
    got = oracle.attention(q, kc, vc, np.array([n - 1]))[0, 0]
    s = (kc[0, :n].astype(np.float64) @ q[0, 0].astype(np.float64)) / math.sqrt(d)
    e = np.exp(s - s.max())
    want = (e / e.sum()) @ vc[0, :n].astype(np.float64)
    assert np.max(np.abs(got - want)) <= 64 * ULP * np.max(np.abs(vc[0, :n])), np.max(np.abs(got - want))


def test_attention_one_key_is_the_value(oracle):
    q = np.ones((1, 2, 16), np.float32)
    kc = np.random.default_rng(0).standard_normal((1, 4, 16)).astype(np.float32)
    vc = np.random.default_rng(1).standard_normal((1, 4, 16)).astype(np.float32)
    got = oracle.attention(q, kc, vc, np.array([0]))
    assert np.array_equal(got[0, 0], vc[0, 0]) and np.array_equal(got[0, 1], vc[0, 0])


def test_attention_weighted_sum_is_ordered_fma(oracle):
    """With the exponentials known, the output is sum_j fma(e_j, v_j, acc)
    in key order divided by the sum: checked against a float32 loop with
    numpy's fused multiply-add emulated through float64 (exact for one
    product and one addend)."""
    d, n = 16, 11
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, d)).astype(np.float32)
    kc = rng.standard_normal((1, n, d)).astype(np.float32)
    vc = rng.standard_normal((1, n, d)).astype(np.float32)
    sc = oracle.scores(q[0, 0], kc[0], np.float32(1.0 / math.sqrt(d)))
    mx = np.float32(sc.max())
    e, tot = oracle.expsum_f32(sc, mx)
    acc = np.zeros(d, np.float32)
    for j in range(n):
        acc = (e[j].astype(np.float64) * vc[0, j].astype(np.float64) + acc.astype(np.float64)).astype(np.float32)
    want = (acc / tot).astype(np.float32)
    got = oracle.attention(q, kc, vc, np.array([n - 1]))[0, 0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def pieces(n, procs):
    w = min(procs, n)
    chunk = n if w <= 1 else max(1, n // (w * 8))
    vec = np.zeros(n, bool)
    for lo in range(0, n, chunk):
        ln = min(chunk, n - lo)
        if ln >= 8:
            vec[lo:lo + (ln & ~7)] = True
    return vec


@pytest.mark.parametrize("n,procs", [(100, 1), (100, 4), (1792, 16), (4096, 7), (5, 16)])
def test_silu_mul(oracle, n, procs):
    """Vector elements within a few ulp of float64 silu(a)*b, tail elements
    of each piece exactly the float64 formula rounded once."""
    rng = np.random.default_rng(n + procs)
    a = (rng.standard_normal(n) * 5).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = oracle.silu_mul(a, b, procs)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    exact = a64 / (1.0 + np.exp(-a64)) * b64
    vec = pieces(n, procs)
    assert np.array_equal(got[~vec], exact[~vec].astype(np.float32))
    rel = np.abs(got[vec] - exact[vec]) / np.maximum(np.abs(exact[vec]), 1e-30)
    assert rel.size == 0 or np.max(rel) <= 6 * ULP, np.max(rel)
