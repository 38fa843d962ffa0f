"""Pins the CPU oracle (oracle/mimref.c) before it is trusted as the checker
of the GPU path: golden vectors and known answers from the reference's own
tests, an exhaustive f16 check, and independent evaluations (exact rational
arithmetic, float64 brute force within the spec's tolerances)."""
import base64
import json
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import GOLDEN
from exact import fma32, i2f32, mul32, round_f32

Q8_0, Q4_K, Q6_K = 64, 66, 67
NAMES = {Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}
U = 2.0 ** -24


def f16(v):
    return np.array([v], np.float16).view(np.uint16)[0]


# ------------------------------------------------------------- f16 / decode

def test_f16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    got = oracle.f16_to_f32(h).view(np.uint32)
    assert np.array_equal(got, want)


def test_f32_to_f16_rounding(oracle):
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(100),
        np.float32([0, -0.0, 65504, 65519.99, 65520, 1e-8, 2 ** -24, 2 ** -25, 3 * 2 ** -26, np.inf, -np.inf]),
        (np.arange(2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2 ** -10),
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.lib().mref_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def _golden():
    return json.load(open(os.path.join(GOLDEN, "quant_golden.json")))


@pytest.mark.parametrize("dt", [Q8_0, Q4_K, Q6_K])
def test_dequantize_golden(oracle, dt):
    """TestDequantizeGolden (reference quant_test.go:285-339)."""
    v = _golden()[NAMES[dt]]
    raw = base64.b64decode(v["bytes"])
    bits = np.array(v["bits"], np.uint32)
    assert np.array_equal(np.array(v["values"], np.float32).view(np.uint32), bits)
    got = oracle.dequantize(dt, raw, bits.size)
    assert np.array_equal(got.view(np.uint32), bits)


def test_dequantize_conformance(oracle):
    cases = json.load(open(os.path.join(GOLDEN, "dequantize_cases.json")))["cases"]
    assert len(cases) == 3
    for c in cases:
        dt = {"q8_0": Q8_0, "q4_k": Q4_K, "q6_k": Q6_K}[c["inputs"][0]["dtype"]]
        raw = bytes.fromhex(c["inputs"][0]["data"])
        want = np.frombuffer(bytes.fromhex(c["output"]["data"]), np.uint32)
        got = oracle.dequantize(dt, raw, want.size)
        assert np.array_equal(got.view(np.uint32), want), c["name"]


def test_dequantize_hand_built(oracle):
    """TestDequantizeHandBuilt (reference quant_test.go:341-477)."""
    blk = bytearray(34)
    blk[0:2] = f16(0.5).tobytes()
    blk[2], blk[33] = 0x7F, 0x80
    y = oracle.dequantize(Q8_0, bytes(blk), 32)
    assert (y[0], y[31], y[1]) == (63.5, -64, 0)

    blk = bytearray(144)
    blk[0:2] = f16(1).tobytes()
    blk[2:4] = f16(0).tobytes()
    for j in range(4):
        blk[4 + j] = j + 1
    for j in range(4, 8):
        v = j + 1
        blk[4 + j + 4] |= v & 0xF
        blk[4 + j - 4] |= (v >> 4) << 6
    for i in range(128):
        blk[16 + i] = 0x11
    y = oracle.dequantize(Q4_K, bytes(blk), 256)
    assert np.array_equal(y, (np.arange(256) // 32 + 1).astype(np.float32))

    blk = bytearray(144)
    blk[0:2] = f16(1).tobytes()
    blk[2:4] = f16(0.5).tobytes()
    blk[4 + 8], blk[4 + 0], blk[4 + 4] = 0x35, 0x80, 0x40
    blk[16 + 64] = 0x02
    y = oracle.dequantize(Q4_K, bytes(blk), 256)
    assert y[128] == np.float32(37 * 2 - 0.5 * 19)
    assert y[129] == np.float32(-0.5 * 19)
    assert y[0] == 0 and y[160] == 0

    blk = bytearray(210)
    blk[208:210] = f16(1).tobytes()
    for i in range(192, 208):
        blk[i] = 1
    blk[0], blk[128], blk[192] = 0xF0, 0x01, 0xFE
    y = oracle.dequantize(Q6_K, bytes(blk), 256)
    assert (y[0], y[64], y[32], y[255]) == (32, -17, -32, -32)


def test_dequantize_errors(oracle):
    """TestDequantizeErrors (reference quant_test.go:500-525): size checks."""
    L = oracle.lib()
    buf = np.zeros(64, np.uint8)
    out = np.zeros(64, np.float32)
    p = lambda a: a.ctypes.data
    assert L.mref_dequantize(Q8_0, p(buf), 34, p(out), 33) < 0
    assert L.mref_dequantize(Q8_0, p(buf), 35, p(out), 32) < 0
    assert L.mref_dequantize(999, p(buf), 0, p(out), 0) < 0
    assert L.mref_dequantize(Q4_K, p(buf), 0, p(out), 0) == 0


def test_q8_0_encoder_matches_gguf(oracle):
    """TestQuantizeMatchesGGUF (reference quant_test.go:542-568)."""
    v = _golden()["q8_0"]
    x = np.array(v["input_bits"], np.uint32).view(np.float32)
    assert np.array_equal(oracle.quantize(Q8_0, x), np.frombuffer(base64.b64decode(v["bytes"]), np.uint8))


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_encoder_round_trip(oracle, dt):
    """The encoders are this repository's own (non-normative): decode(encode(x))
    must be within one quantization step of x."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(256 * 16).astype(np.float32) * np.float32(0.02)
    y = oracle.dequantize(dt, oracle.quantize(dt, x), x.size)
    step = {Q4_K: 2 * 0.02 * 4 / 15, Q6_K: 0.02 * 4 / 31, Q8_0: 0.02 * 4 / 127}[dt]
    assert np.max(np.abs(x - y)) < step
    # and it is far from trivially zero
    assert np.corrcoef(x, y)[0, 1] > 0.98


# ------------------------------------------------------- activation quantizer

def test_quantize_act_known_answers(oracle):
    """TestQuantQ8 / TestQuantizeQ8Rejects (reference q8_test.go:58-107)."""
    y = np.zeros(32, np.float32)
    y[:3] = [254, 1, 3]
    a = oracle.Act(y, 32)
    assert a.ok and list(a.q[:3]) == [127, 0, 2]
    for bad in (np.inf, np.nan, 1e30, -np.inf):
        y[5] = bad
        assert not oracle.Act(y, 32).ok
        z = np.random.default_rng(15).standard_normal(512).astype(np.float32)
        z[300] = bad
        assert not oracle.Act(z, 256).ok
    z = np.random.default_rng(1).standard_normal(512).astype(np.float32)
    z[300] = 40
    a = oracle.Act(z, 256)
    assert a.ok and a.q[300] == 127
    assert np.all(a.d[8:16] == np.float32(40.0) / np.float32(127))
    assert not oracle.Act(np.zeros(288, np.float32), 256).ok
    assert not oracle.Act(np.zeros(48, np.float32), 32).ok
    # 2^60 is accepted, the next float above is refused
    w = np.zeros(256, np.float32)
    w[7] = 2.0 ** 60
    assert oracle.Act(w, 256).ok
    w[7] = np.nextafter(np.float32(2.0 ** 60), np.float32(np.inf))
    assert not oracle.Act(w, 256).ok


@pytest.mark.parametrize("block", [32, 256])
def test_quantize_act_exact_rounding(oracle, block):
    """q = RoundToEven(127 x / amax) with the exact quotient (q8.go:78-84), d =
    amax/127 rounded once, xs and m32 the integer sums; checked with rationals."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(512).astype(np.float32)
    # values near half-integer steps, where the rounding matters
    amax = np.float32(np.max(np.abs(x[:block])))
    for j, t in enumerate([0.5, 1.5, 2.5, 3.5000002, 10.499999, -0.5, -7.5]):
        x[1 + j] = np.float32(t * float(amax) / 127.0)
    x[400:400 + 32] = 0  # a zero run (a zero block when block == 32)
    a = oracle.Act(x, block)
    assert a.ok
    for b in range(x.size // block):
        xb = x[block * b:block * (b + 1)]
        am = max(abs(Fraction(float(v))) for v in xb)
        for i, v in enumerate(xb):
            if am == 0:
                want = 0
            else:
                t = Fraction(127) * Fraction(float(v)) / am
                n = t.numerator // t.denominator
                r = t - n
                want = n + (1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2)) else 0)
            assert a.q[block * b + i] == want
        d = round_f32(am / 127)
        assert np.all(a.d[block * b // 32:block * (b + 1) // 32] == d)
    for r in range(x.size // 32):
        s = int(a.q[32 * r:32 * r + 32].astype(np.int32).sum())
        assert a.xs[r] == s
        assert a.dbs[r] == mul32(a.d[r], np.float32(s))
    for i in range(x.size // 2):
        assert a.m32[i] == 32 * (int(a.q[2 * i]) + int(a.q[2 * i + 1]))


# ------------------------------------------------ block-256 8-bit dot product

def q4k_scale_min(s, j):
    """getScaleMinK4 as spec/dtypes.md:187-196 states it."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def f16val(b):
    return np.frombuffer(bytes(b), np.float16)[0].astype(np.float32)


def ref_dot_a8k(dt, row, act):
    """dotQ8KRef (reference q8k_test.go:38-102) with exact integers and an
    exactly rounded FMA (big rationals), independent of any hardware FMA."""
    tot = off = np.float32(0)
    row = bytes(row)
    for b in range(act.k // 256):
        y = [int(v) for v in act.q[256 * b:256 * b + 256]]
        dx = act.d[8 * b]
        if dt == Q4_K:
            blk = row[144 * b:144 * b + 144]
            if (blk[1] & 0x7C) == 0x7C or (blk[3] & 0x7C) == 0x7C:
                return None
            d, dmin = f16val(blk[0:2]), f16val(blk[2:4])
            S = M = 0
            for j in range(8):
                sc, m = q4k_scale_min(blk[4:16], j)
                c, hi = j // 2, j % 2
                qs = [(blk[16 + 32 * c + i] >> (4 * hi)) & 15 for i in range(32)]
                S += sc * sum(q * yy for q, yy in zip(qs, y[32 * j:32 * j + 32]))
                M += m * int(act.xs[8 * b + j])
            tot = fma32(i2f32(S), mul32(d, dx), tot)
            off = fma32(i2f32(M), mul32(dmin, dx), off)
        else:
            blk = row[210 * b:210 * b + 210]
            if (blk[209] & 0x7C) == 0x7C:
                return None
            d = f16val(blk[208:210])
            S = 0
            for e in range(256):
                h, r = divmod(e, 128)
                p, l = divmod(r, 32)
                ql, qh = blk[64 * h:64 * h + 64], blk[128 + 32 * h:160 + 32 * h]
                lo = ql[l + 32 * (p % 2)]
                lo = (lo & 15) if p < 2 else (lo >> 4)
                q = lo | (((qh[l] >> (2 * p)) & 3) << 4)
                sb = blk[192 + 8 * h + l // 16 + 2 * p]
                sc = sb - 256 if sb >= 128 else sb
                S += sc * (q - 32) * y[e]
            tot = fma32(i2f32(S), mul32(d, dx), tot)
    return np.float32(tot - off)


def _acts(oracle, k, n=5, seed=14):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        x = rng.standard_normal(k).astype(np.float32)
        if i == 1:
            x *= np.float32(1e-30)
        elif i == 2:
            x *= np.float32(1e15)
        elif i == 3:
            x[:256] = 0
        a = oracle.Act(x, 256)
        assert a.ok
        out.append(a)
    return out


def _special_rows(dt, k, trial, rng, oracle):
    row = bytearray(oracle.synthetic_weight(dt, 1, k, seed=int(rng.integers(1 << 30))).tobytes())
    if dt == Q4_K:
        if trial == 1:  # largest finite scales, all-ones quants (q8k_test.go:137-155)
            for o in range(0, len(row), 144):
                row[o:o + 4] = b"\xff\x7b\xff\x7b"
                row[o + 4:o + 144] = b"\xff" * 140
        if trial == 2:  # subnormal f16 scales
            row[0:4] = b"\x01\x00\xff\x03"
    else:
        if trial == 1:
            for o in range(0, len(row), 210):
                row[o + 208:o + 210] = b"\xff\x7b"
                row[o:o + 192] = b"\xff" * 192
                row[o + 192:o + 208] = b"\x80" * 16
        if trial == 2:
            row[208:210] = b"\x01\x00"
    return bytes(row)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
@pytest.mark.parametrize("k", [256, 2048])
def test_dot_a8k_closed_form(oracle, dt, k):
    """TestDotQ8KReference's inputs (q8k_test.go:104-187): the oracle equals
    the exactly evaluated closed form bit for bit."""
    rng = np.random.default_rng(k + dt)
    acts = _acts(oracle, k)
    for trial in range(3):
        row = _special_rows(dt, k, trial, rng, oracle)
        for a in acts:
            got = oracle.dot_a8(dt, np.frombuffer(row, np.uint8), a)
            want = ref_dot_a8k(dt, row, a)
            assert got is not None and want is not None
            assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), (trial, got, want)


def test_dot_a8k_llama_blocks(oracle):
    """Blocks written by llama.cpp's quantizer (reference testdata/llama):
    the oracle equals the exact closed form bit for bit."""
    z = np.load(os.path.join(GOLDEN, "llama_tensors.npz"))
    rng = np.random.default_rng(2)
    for name in ("blk_0_attn_q_weight", "blk_0_ffn_down_weight", "output_weight", "blk_1_attn_v_weight"):
        raw, shape, dt = z[name + "__bytes"], z[name + "__shape"], int(z[name + "__dtype"][0])
        n, k = int(shape[0]), int(shape[1])
        rb = raw.size // n
        a = oracle.Act(rng.standard_normal(k).astype(np.float32), 256)
        for j in range(0, n, max(1, n // 6)):
            row = raw[rb * j:rb * (j + 1)]
            got = oracle.dot_a8(dt, row, a)
            want = ref_dot_a8k(dt, row.tobytes(), a)
            assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32)


@pytest.mark.parametrize("dt", [Q4_K, Q6_K])
def test_dot_a8k_refuses_nonfinite_scales(oracle, dt):
    k = 512
    a = _acts(oracle, k, n=1)[0]
    row = bytearray(oracle.synthetic_weight(dt, 1, k, seed=1).tobytes())
    assert oracle.dot_a8(dt, np.frombuffer(bytes(row), np.uint8), a) is not None
    base = 210 if dt == Q6_K else 144  # the second block
    for f in ([208] if dt == Q6_K else [0, 2]):
        r = bytearray(row)
        r[base + f:base + f + 2] = b"\x00\x7c"  # +inf (d, or dmin of Q4_K)
        assert oracle.dot_a8(dt, np.frombuffer(bytes(r), np.uint8), a) is None


def _wd_terms(dt, row_bytes, k, oracle):
    """The reference decode and B_jk of spec/stdlib.md:251-268."""
    wd = oracle.dequantize(dt, row_bytes, k).astype(np.float64)
    if dt != Q4_K:
        return wd, np.abs(wd)
    B = np.zeros(k)
    for b in range(k // 256):
        blk = row_bytes[144 * b:144 * b + 144]
        d, dmin = float(f16val(blk[0:2])), float(f16val(blk[2:4]))
        for j in range(8):
            sc, m = q4k_scale_min(blk[4:16], j)
            c, hi = j // 2, j % 2
            q = np.array([(blk[16 + 32 * c + i] >> (4 * hi)) & 15 for i in range(32)], np.float64)
            B[256 * b + 32 * j:256 * b + 32 * j + 32] = np.abs(d * sc * q) + abs(dmin * m)
    return wd, B


@pytest.mark.parametrize("dt,block", [(Q4_K, 256), (Q6_K, 256), (Q8_0, 32), (Q4_K, 32), (Q6_K, 32)])
def test_dot_a8_within_spec_tolerance(oracle, dt, block):
    """dequant_matmul_a8 tolerance (spec/stdlib.md:251-279) against a float64
    brute force of the reference decode: independent of the kernels' order."""
    k = 2048
    rng = np.random.default_rng(7)
    wbytes = oracle.synthetic_weight(dt, 4, k, seed=3)
    rb = wbytes.size // 4
    for i in range(3):
        x = rng.standard_normal(k).astype(np.float32) * np.float32(10.0 ** (i - 1))
        a = oracle.Act(x, block)
        s = np.repeat(np.abs(x.reshape(-1, block)).max(1) / 127.0, block).astype(np.float64)
        for j in range(4):
            row = wbytes[rb * j:rb * (j + 1)]
            got = float(oracle.dot_a8(dt, row, a))
            wd, B = _wd_terms(dt, row.tobytes(), k, oracle)
            exact = float(np.dot(x.astype(np.float64), wd))
            tol = (k + 2) * U * float(np.sum((np.abs(x) + s) * B)) + float(np.sum(s * np.abs(wd)))
            assert abs(got - exact) <= tol, (got, exact, tol)


# ------------------------------------------------------ float32 dot products

@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_f32_dot_decodes_exactly(oracle, dt):
    """TestRowDotDecodesExactly (reference kernels_test.go:119-139): with a
    unit vector the fused kernel returns the decoded weight exactly."""
    k = 512
    row = oracle.synthetic_weight(dt, 1, k, seed=9)
    wd = oracle.dequantize(dt, row, k)
    for e in list(range(0, k, 37)) + [k - 1]:
        x = np.zeros(k, np.float32)
        x[e] = 1
        assert oracle.dot_f32(dt, row, x) == wd[e]
        assert oracle.dot_plain_f32(x, wd) == wd[e]


@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_f32_dot_within_spec_tolerance(oracle, dt):
    """linear.v1 / dequant_matmul.v1 tolerance (K+1) u sum|x w| (spec/stdlib.md:225-244)."""
    k = 4096
    rng = np.random.default_rng(8)
    wbytes = oracle.synthetic_weight(dt, 3, k, seed=4)
    rb = wbytes.size // 3
    for j in range(3):
        row = wbytes[rb * j:rb * (j + 1)]
        x = rng.standard_normal(k).astype(np.float32)
        wd = oracle.dequantize(dt, row, k).astype(np.float64)
        exact = float(np.dot(x.astype(np.float64), wd))
        tol = (k + 1) * U * float(np.sum(np.abs(x * wd)))
        for got in (oracle.dot_f32(dt, row, x), oracle.dot_plain_f32(x, wd.astype(np.float32))):
            assert abs(float(got) - exact) <= tol


# -------------------------------------------------------------- the drivers

def test_linear_a8_fallbacks_and_bias(oracle):
    """linearA8 (reference interp/fast.go:282-379): refused rows of x and
    rows of w with a non-finite scale take the float32 path; bias is added."""
    n, k, rows = 6, 512, 5
    w = bytearray(oracle.synthetic_weight(Q4_K, n, k, seed=2).tobytes())
    rb = len(w) // n
    w[rb * 3 + 1] = 0x7C  # row 3: d = inf in its first block (high byte)
    w[rb * 3 + 0] = 0x00
    w = np.frombuffer(bytes(w), np.uint8)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[2, 17] = np.nan
    bias = rng.standard_normal(n).astype(np.float32)
    y = oracle.linear_a8(x, w, Q4_K, n, k, bias=bias, block=256)
    for i in range(rows):
        for j in range(n):
            row = w[rb * j:rb * (j + 1)]
            a = oracle.Act(x[i], 256)
            s = oracle.dot_a8(Q4_K, row, a) if a.ok else None
            if s is None:
                s = oracle.dot_f32(Q4_K, row, x[i])
            want = np.float32(s + bias[j])
            assert y[i, j].view(np.uint32) == want.view(np.uint32) or (np.isnan(y[i, j]) and np.isnan(want))
    assert np.isnan(y[2]).all()
    # Q8_0 with blocks of 256 has no 8-bit kernel: the float32 path
    w8 = oracle.synthetic_weight(Q8_0, n, k, seed=5)
    y8 = oracle.linear_a8(x[:2], w8, Q8_0, n, k, block=256)
    assert np.array_equal(y8, oracle.linear_f32(x[:2], w8, Q8_0, n, k))


def test_linear_threads_do_not_change_bits(oracle):
    n, k, rows = 64, 1024, 3
    w = oracle.synthetic_weight(Q6_K, n, k, seed=6)
    x = np.random.default_rng(4).standard_normal((rows, k)).astype(np.float32)
    y1 = oracle.linear_a8(x, w, Q6_K, n, k, threads=1)
    y4 = oracle.linear_a8(x, w, Q6_K, n, k, threads=4)
    assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))
