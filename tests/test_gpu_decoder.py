"""The decoder step on the GPU (mimir-model_amd/decoder.py over libmimg's
decoder ops) against the reference's fixtures and the CPU restatement.

Op by op: attention and swiglu follow the operation order of the
reference's AVX2 kernels and are compared with the C restatement bit for
bit; the integer ops (embedding rows, the cache scatter, argmax, the greedy
step) are exact; rms_norm and rope, whose only inexact steps are f64 (a sum
of squares, cos/sin), within one f32 rounding. End to end, the checks are
the reference's own (cmd/mim-run/main_test.go:178-257): 2e-5 of the largest
logit and the same greedy ids without 8-bit activations, llama.cpp's
deviation from the float64 oracle (x1.1 with the cache in f16) with them;
and the same greedy ids as the CPU restatement with them."""
import json
import os
import sys

import numpy as np
import pytest

import fixture_models as fm
import llama_ref

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 64, 66, 67


@pytest.fixture(scope="module")
def rt(gpu):
    import hiprt

    return hiprt


def dev(rt, a):
    return rt.DeviceBuffer.from_array(np.ascontiguousarray(a))


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


# ------------------------------------------------------------ single ops

@pytest.mark.parametrize("dt", [Q4_K, Q6_K, Q8_0])
def test_embedding_rows_exact(gpu, oracle, rt, dt):
    V, E = 37, 512
    raw = oracle.synthetic_weight(dt, V, E, seed=3)
    w = gpu.Weight(raw, dt, V, E)
    # ids outside 0..V-1 give zero rows, as the reference leaves them
    # (interp/fast.go:834-838)
    ids = np.array([0, 5, 36, -1, 5, V, 17], np.int32)
    s = rt.Stream()
    d_ids, out = dev(rt, ids), rt.DeviceBuffer(ids.size * E * 4)
    out.upload(np.full(ids.size * E, np.nan, np.float32))
    gpu.embedding_dev(w, d_ids.ptr, ids.size, out.ptr, s.handle)
    s.sync()
    got = out.download(np.float32).reshape(ids.size, E)
    rb = len(raw) // V
    for i, t in enumerate(ids):
        if 0 <= t < V:
            want = oracle.dequantize(dt, raw[rb * t: rb * (t + 1)], E)
        else:
            want = np.zeros(E, np.float32)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"row {i} (token {t})"
    w.release()


@pytest.mark.parametrize("rows,n,resid", [(1, 256, False), (7, 2048, True), (3, 4096, True), (2, 100, False)])
def test_rms_norm(gpu, rt, rows, n, resid):
    rng = np.random.default_rng(n + rows)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    r = rng.standard_normal((rows, n)).astype(np.float32)
    sc = rng.standard_normal(n).astype(np.float32)
    s = rt.Stream()
    dx, dr, dsc, dy = dev(rt, x), dev(rt, r), dev(rt, sc), rt.DeviceBuffer(x.nbytes)
    gpu.rms_norm_dev(dx.ptr, dr.ptr if resid else None, dsc.ptr, 1e-5, rows, n, dy.ptr, s.handle)
    s.sync()
    xr = (x + r).astype(np.float32) if resid else x
    # the residual add is one f32 add: exact
    assert np.array_equal(dx.download(np.float32).reshape(rows, n), xr)
    want = llama_ref.rms_norm(xr, sc, 1e-5)
    got = dy.download(np.float32).reshape(rows, n)
    # f64 sum of squares in another order: inv may differ in its last bit
    assert rel_err(got, want) <= 2e-7, rel_err(got, want)


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope(gpu, rt, interleaved):
    T, H, D, rot, theta = 5, 8, 64, 64, 500000.0
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([0, 1, 7, 300, 4095], np.int64)
    invf = np.array([theta ** (-2.0 * i / rot) for i in range(rot // 2)], np.float64)
    s = rt.Stream()
    dx, dp, di = dev(rt, x), dev(rt, pos), dev(rt, invf)
    gpu.rope_dev(dx.ptr, dp.ptr, di.ptr, T, H, D, rot, interleaved, s.handle)
    s.sync()
    cos, sin = llama_ref.rope_tables(pos, rot, theta)
    want = llama_ref.rope(x, cos, sin, rot, interleaved)
    got = dx.download(np.float32).reshape(T, H, D)
    # f64 cos/sin of the device library vs numpy's, rounded to f32: a last-bit
    # difference in c or s at most
    assert np.max(np.abs(got - want)) <= 4e-7 * np.max(np.abs(x)) * 2, np.max(np.abs(got - want))


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("T,H,Hkv,D,slots", [(1, 32, 8, 64, 1), (6, 4, 2, 64, 1), (3, 8, 8, 128, 2), (4, 4, 1, 32, 3),
                                             (5, 2, 1, 8, 1), (2, 4, 2, 256, 1)])
def test_kv_store_and_attention_bitexact(gpu, oracle, rt, f16, T, H, Hkv, D, slots, C=48):
    """The cache scatter (exact) and attention against the C restatement of
    the reference's attendRow with its AVX2 kernels, bit for bit; visible
    ranges of every length mod 4 and mod 8 (the scores' groups of four and
    the exp sum's vector part and tail)."""
    rng = np.random.default_rng(T * 100 + H + D)
    L = slots * C
    # a cache already holding rows, then T new rows at the given positions
    cdt = np.float16 if f16 else np.float32
    base = (rng.standard_normal((2, Hkv, L, D)) * 2).astype(cdt)
    slot = np.arange(T) % slots
    pos = np.array([C - 1 - 2 * i if i % 2 else 3 + 5 * i for i in range(T)], np.int64)
    cidx = slot * C + pos
    k = (rng.standard_normal((T, Hkv, D)) * 2).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    kc, vc = dev(rt, base[0]), dev(rt, gpu.pack_vcache(base[1]))  # the value cache blocked by 8 keys
    dk, dv, dq, dc, ds = dev(rt, k), dev(rt, v), dev(rt, q), dev(rt, cidx), dev(rt, (slot * C).astype(np.int64))
    out = rt.DeviceBuffer(q.nbytes)
    wsb = gpu.attention_workspace_bytes(T, H, C)
    ws = rt.DeviceBuffer(wsb)
    s = rt.Stream()
    gpu.kv_store_dev(dk.ptr, dv.ptr, dc.ptr, T, Hkv, D, L, kc.ptr, vc.ptr, f16, s.handle)
    gpu.attention_dev(dq.ptr, kc.ptr, vc.ptr, dc.ptr, ds.ptr if slots > 1 else None, T, H, Hkv, D, L, C, f16, out.ptr,
                      ws.ptr, wsb, s.handle)
    s.sync()
    wk, wv = base[0].copy(), base[1].copy()
    for t in range(T):
        wk[:, cidx[t]] = k[t]  # rounded to f16 (RNE) with an f16 cache
        wv[:, cidx[t]] = v[t]
    got_k = kc.download(cdt).reshape(Hkv, L, D)
    got_v = gpu.unpack_vcache(vc.download(cdt), Hkv, L, D)
    assert np.array_equal(got_k.view(np.uint16 if f16 else np.uint32), wk.view(np.uint16 if f16 else np.uint32))
    assert np.array_equal(got_v.view(np.uint16 if f16 else np.uint32), wv.view(np.uint16 if f16 else np.uint32))
    want = oracle.attention(q, wk, wv, cidx, slot * C if slots > 1 else None)
    got = out.download(np.float32).reshape(T, H, D)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), float(np.max(np.abs(got - want)))


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("C,D", [(700, 128), (1100, 64), (300, 8), (250, 128), (256, 64)])
def test_attention_long_context_bitexact(gpu, oracle, rt, f16, C, D):
    """Long visible ranges: many score tiles and several value chunks."""
    test_kv_store_and_attention_bitexact(gpu, oracle, rt, f16, 3, 4, 2, D, 1, C=C)


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("T,H,Hkv,D,slots,C", [(2, 32, 8, 128, 2, 1100), (3, 16, 2, 64, 1, 3000), (8, 32, 8, 128, 8, 300),
                                               (4, 8, 4, 64, 2, 1100), (1, 32, 8, 128, 1, 2100),
                                               (2, 32, 8, 128, 2, 400), (4, 16, 2, 64, 2, 600),
                                               (2, 4, 4, 128, 1, 300), (3, 8, 4, 64, 1, 700), (1, 32, 8, 128, 1, 768)])
def test_attention_grouped_heads_bitexact(gpu, oracle, rt, f16, T, H, Hkv, D, slots, C):
    """Past 256 keys at few queries, when tiles x kv heads x queries reaches
    256 workgroups, the scores of the query heads that share a kv head come
    from one workgroup (groups of 2, 4 and 8 heads, slots, the 8B decode
    shape at 768 keys; one head per kv head and short grids stay per head):
    bit for bit the restatement."""
    test_kv_store_and_attention_bitexact(gpu, oracle, rt, f16, T, H, Hkv, D, slots, C=C)


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("T,H,Hkv,D,C,sign", [(2, 32, 8, 128, 300, 1), (3, 8, 2, 64, 520, -1), (1, 8, 2, 128, 700, 1)])
def test_attention_nonfinite_key(gpu, oracle, rt, f16, T, H, Hkv, D, C, sign):
    """A key with an infinite element in one kv head: that key's scores are
    +inf (its query heads give NaN) or -inf (its exponential is 0 and the
    heads stay finite), as the reference computes them; every other head
    keeps the restatement's bits."""
    rng = np.random.default_rng(T * 7 + H + D + C)
    cdt = np.float16 if f16 else np.float32
    wk = (rng.standard_normal((Hkv, C, D)) * 2).astype(cdt)
    wv = rng.standard_normal((Hkv, C, D)).astype(cdt)
    wk[1, 5, 3] = sign * np.inf
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    q[:, :, 3] = np.abs(q[:, :, 3]) + 0.25  # the key's scores are sign * inf in every head of kv head 1
    cidx = np.array([C - 1 - 3 * t for t in range(T)], np.int64)
    kc, vc = dev(rt, wk), dev(rt, gpu.pack_vcache(wv))
    dq, dc = dev(rt, q), dev(rt, cidx)
    out = rt.DeviceBuffer(q.nbytes)
    wsb = gpu.attention_workspace_bytes(T, H, C)
    ws = rt.DeviceBuffer(wsb)
    s = rt.Stream()
    gpu.attention_dev(dq.ptr, kc.ptr, vc.ptr, dc.ptr, None, T, H, Hkv, D, C, C, f16, out.ptr, ws.ptr, wsb, s.handle)
    s.sync()
    want = oracle.attention(q, wk, wv, cidx, None)
    got = out.download(np.float32).reshape(T, H, D)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    G = H // Hkv
    if sign > 0:  # the largest score is +inf: NaN
        assert np.isnan(got[:, G:2 * G]).all()
    else:  # -inf: the key's exponential is 0
        assert not np.isnan(got).any()
    assert not np.isnan(got[:, :G]).any()


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("T,H,Hkv,D,C", [(5, 4, 1, 64, 42), (4, 8, 2, 128, 45), (5, 4, 2, 32, 42), (3, 4, 2, 128, 301)])
def test_attention_unaligned_slots_bitexact(gpu, oracle, rt, f16, T, H, Hkv, D, C):
    """Three slots of C entries with C not a multiple of 8: the visible ranges
    start inside an 8-key block of the value cache (the weighted sum skips
    the keys before them, one at a time), through the short-context kernel
    (D = 64/128, C <= 256) and the two-kernel path (D = 32, C = 301)."""
    test_kv_store_and_attention_bitexact(gpu, oracle, rt, f16, T, H, Hkv, D, 3, C=C)


@pytest.mark.parametrize("n,procs", [(3 * 8192 + 5, 16), (1792, 16), (100, 4), (100, 1), (4096, 7), (7, 16)])
def test_swiglu_bitexact(gpu, oracle, rt, n, procs):
    """swiglu against the restatement of SiluMulF32 over the reference's
    pieces for GOMAXPROCS = procs, bit for bit (pieces with and without an
    f64 tail)."""
    rng = np.random.default_rng(5 + n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:4] = [0.0, -0.0, 90.0, -200.0]
    u = rng.standard_normal(n).astype(np.float32)
    s = rt.Stream()
    dg, du, do = dev(rt, g), dev(rt, u), rt.DeviceBuffer(g.nbytes)
    gpu.swiglu_dev(dg.ptr, du.ptr, do.ptr, n, procs, s.handle)
    s.sync()
    want = oracle.silu_mul(g, u, procs)
    got = do.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int(np.sum(got.view(np.uint32) != want.view(np.uint32)))


def test_argmax_first_index(gpu, rt):
    rows, n = 4, 128256
    rng = np.random.default_rng(9)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[1, 77] = x[1, 100000] = 50.0   # tie: the first index wins
    x[2, :] = -1.0                    # all equal
    x[3, n - 1] = 60.0
    s = rt.Stream()
    dx, do = dev(rt, x), rt.DeviceBuffer(rows * 4)
    gpu.argmax_dev(dx.ptr, rows, n, do.ptr, s.handle)
    s.sync()
    got = do.download(np.int32)
    assert got.tolist() == [int(np.argmax(r)) for r in x] == [got[0], 77, 0, n - 1]
    # the reference's loop (best = 0; x > v[best]): NaNs are never chosen,
    # a NaN first value gives 0; odd lengths (unaligned rows)
    y = rng.standard_normal((3, 1001)).astype(np.float32)
    y[0, 5] = np.nan
    y[1, 0] = np.nan
    y[2, :] = np.nan
    dy, dz = dev(rt, y), rt.DeviceBuffer(3 * 4)
    gpu.argmax_dev(dy.ptr, 3, 1001, dz.ptr, s.handle)
    s.sync()
    want0 = int(np.nanargmax(y[0]))
    assert dz.download(np.int32).tolist() == [want0, 0, 0]
    # aligned rows (whole float4s): NaNs inside the float4 of the maximum, a
    # tie inside one float4, all -inf, +inf twice, a NaN first value
    z = rng.standard_normal((6, n)).astype(np.float32)
    z[0, 4000:4004] = [np.nan, 3.0, 70.0, np.nan]
    z[1, 808:812] = [1.0, 80.0, 2.0, 80.0]
    z[2, :] = -np.inf
    z[3, 99] = z[3, 60001] = np.inf
    z[4, 0] = np.nan
    z[4, 5000] = 90.0
    z[5, 1::2] = np.nan
    z[5, 20002] = 75.0

    def ref(row):  # the reference's loop: best = 0, then x[i] > x[best]
        if np.isnan(row[0]):
            return 0
        return int(np.flatnonzero(row == np.nanmax(row))[0])

    dzz, dzo = dev(rt, z), rt.DeviceBuffer(6 * 4)
    gpu.argmax_dev(dzz.ptr, 6, n, dzo.ptr, s.handle)
    s.sync()
    got = dzo.download(np.int32).tolist()
    assert got == [ref(r) for r in z] == [4002, 809, 0, 99, 0, 20002]


def test_greedy_advance(gpu, rt):
    n, cap = 3, 2
    s = rt.Stream()
    chosen = dev(rt, np.array([4, 5, 6], np.int32))
    ids, pos, cidx = dev(rt, np.zeros(n, np.int32)), dev(rt, np.array([1, 2, 3], np.int64)), dev(rt, np.array([10, 20, 30], np.int64))
    out, count = dev(rt, np.full(cap * n, -1, np.int32)), dev(rt, np.zeros(1, np.int32))
    for _ in range(3):  # the third step is past cap: not stored
        gpu.greedy_advance_dev(chosen.ptr, ids.ptr, pos.ptr, cidx.ptr, out.ptr, count.ptr, cap, n, s.handle)
    s.sync()
    assert ids.download(np.int32).tolist() == [4, 5, 6]
    assert pos.download(np.int64).tolist() == [4, 5, 6]
    assert cidx.download(np.int64).tolist() == [13, 23, 33]
    assert out.download(np.int32).tolist() == [4, 5, 6, 4, 5, 6]
    assert count.download(np.int32).tolist() == [3]


# ------------------------------------------------------------ end to end

def gpu_steps(name, a8, cache_f16):
    import decoder

    cfg, tensors, e = fm.load(name)
    dec = decoder.Decoder(cfg, tensors, a8=a8, cache_f16=cache_f16, max_rows=16)
    P = len(e["prompt_ids"])
    prompt = dec.forward(e["prompt_ids"], np.arange(P))
    steps = [prompt[-1]]
    for i, tok in enumerate(e["greedy"][:-1]):
        steps.append(dec.forward([tok], [P + i])[0])
    return dec, e, prompt, steps


@pytest.mark.parametrize("name", fm.FIXTURES)
def test_fixture_generate_f32(gpu, name):
    """TestGenerateMatchesOracle on the GPU: the float32 fast paths, every
    logit within 2e-5 of the largest, the oracle's greedy ids, and the same
    ids from the graph-replayed generate loop."""
    dec, e, prompt, steps = gpu_steps(name, a8=False, cache_f16=False)
    ok, worst, allowed = fm.near(prompt, fm.f32b64(e["prompt_logits"]), 2e-5)
    assert ok, f"prompt logits: {worst} > {allowed}"
    for i, lg in enumerate(steps):
        ok, worst, allowed = fm.near(lg, fm.f32b64(e["greedy_logits"][i]), 2e-5)
        assert ok, f"step {i}: {worst} > {allowed}"
        assert int(np.argmax(lg)) == e["greedy"][i], f"step {i}"
    dec.reset()
    got = dec.generate([e["prompt_ids"]], len(e["greedy"]))
    assert got[0].tolist() == e["greedy"]


@pytest.mark.parametrize("name", fm.FIXTURES)
def test_fixture_generate_f32_matrix_cores(gpu, name):
    """The float32 path with every product on the fp32 matrix cores
    (f32_tile_rows=1: dequant_matmul.v1 within the spec's bound, another
    summation order): every logit still within 2e-5 of the largest of the
    Go executor's, and its greedy ids."""
    import decoder

    cfg, tensors, e = fm.load(name)
    dec = decoder.Decoder(cfg, tensors, a8=False, max_rows=16, f32_tile_rows=1)
    P = len(e["prompt_ids"])
    prompt = dec.forward(e["prompt_ids"], np.arange(P))
    ok, worst, allowed = fm.near(prompt, fm.f32b64(e["prompt_logits"]), 2e-5)
    assert ok, f"prompt logits: {worst} > {allowed}"
    lg = prompt[-1]
    for i, tok in enumerate(e["greedy"]):
        ok, worst, allowed = fm.near(lg, fm.f32b64(e["greedy_logits"][i]), 2e-5)
        assert ok, f"step {i}: {worst} > {allowed}"
        assert int(np.argmax(lg)) == tok, f"step {i}"
        if i + 1 < len(e["greedy"]):
            lg = dec.forward([tok], [P + i])[0]


@pytest.mark.parametrize("cache_f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("name", fm.FIXTURES)
def test_fixture_generate_a8(gpu, name, cache_f16):
    """TestGenerateA8 on the GPU: within llama.cpp's deviation (x1.1 with the
    cache in f16); and the greedy ids of generate() equal the CPU
    restatement's picks with the same numerics."""
    dec, e, prompt, steps = gpu_steps(name, a8=True, cache_f16=cache_f16)
    worst = fm.max_diff(prompt, fm.f32b64(e["prompt_logits"]))
    for i, lg in enumerate(steps):
        worst = max(worst, fm.max_diff(lg, fm.f32b64(e["greedy_logits"][i])))
    bound = e["llama_cpp_max_diff"] * (1.1 if cache_f16 else 1.0)
    assert worst <= bound, f"max |logit difference| {worst} > {bound}"
    cfg, tensors, _ = fm.load(name)
    ref = llama_ref.Decoder(llama_ref.Model(cfg, tensors), a8=True, cache_f16=cache_f16, threads=4)
    P, n = len(e["prompt_ids"]), 12
    lg = ref.forward(e["prompt_ids"], np.arange(P))[-1]
    want = []
    for i in range(n):
        want.append(llama_ref.argmax(lg))
        lg = ref.forward([want[-1]], [P + i])[0]
    dec.reset()
    assert dec.generate([e["prompt_ids"]], n)[0].tolist() == want


def test_slots_match_single_sequences(gpu):
    """Three prompts in three slots of one cache, decoded as a batch of
    rows, give each prompt's own greedy continuation."""
    import decoder

    cfg, tensors, e = fm.load("llama")
    rng = np.random.default_rng(1)
    prompts = rng.integers(1, 400, (3, 6)).astype(np.int32)
    batch = decoder.Decoder(cfg, tensors, a8=True, max_rows=32, slots=3)
    got = batch.generate(prompts, 10)
    single = decoder.Decoder(cfg, tensors, a8=True, max_rows=32, slots=1)
    for i in range(3):
        single.reset()
        assert single.generate(prompts[i:i + 1], 10)[0].tolist() == got[i].tolist(), f"slot {i}"


def test_graph_replay_equals_eager(gpu):
    """The captured decode step replayed gives the same ids as the same
    calls made one by one."""
    import decoder

    cfg, tensors, e = fm.load("qwen2")
    dec = decoder.Decoder(cfg, tensors, a8=True, max_rows=16)
    a = dec.generate([e["prompt_ids"]], 20, graph=True)
    dec.reset()
    b = dec.generate([e["prompt_ids"]], 20, graph=False)
    assert a.tolist() == b.tolist()


def _oracle_greedy(ref, prompt, n_new):
    """Greedy ids of the CPU restatement (reference cmd/mim-run/main.go
    generate, 184-257): the prompt's last logits, then one token a step."""
    P = len(prompt)
    lg = ref.forward(prompt, np.arange(P))[-1]
    want = []
    for i in range(n_new):
        want.append(llama_ref.argmax(lg))
        if i + 1 < n_new:
            lg = ref.forward([want[-1]], [P + i])[0]
    return want


@pytest.mark.parametrize("cache_f16", [False, True], ids=["f32cache", "f16cache"])
def test_llama1b_shape_greedy_matches_oracle(gpu, cache_f16):
    """the Llama-3.2-1B model shape (16 layers, d 2048,
    FFN 8192, 32/8 heads, vocab 128256) with random Q4_K_M weights built on
    the device, a 32-token prompt (uniform ids, seed 7) and all 128 greedy
    tokens of the config; the GPU decoder and the CPU restatement, on the
    same weight bytes, pick the same ids."""
    import decoder
    import synthetic

    cfg = dict(synthetic.LLAMA_1B, context=192)
    tensors = synthetic.build(cfg, seed=1)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 32).astype(np.int32)
    n_new = 128
    dec = decoder.Decoder(cfg, tensors, a8=True, cache_f16=cache_f16, max_rows=32)
    got = dec.generate([prompt], n_new)[0].tolist()
    del dec
    ref = llama_ref.Decoder(llama_ref.Model(cfg, synthetic.host_bytes(tensors)), a8=True, cache_f16=cache_f16,
                            threads=16)
    want = _oracle_greedy(ref, prompt, n_new)
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


@pytest.fixture(scope="module")
def llama8b(gpu):
    """BASELINE config 4's model: the Llama-3-8B shape (32 layers, d 4096,
    FFN 14336, 32/8 heads, vocab 128256) with random Q4_K_M weights drawn
    and encoded on the device (4.9 GB)."""
    import synthetic

    cfg = dict(synthetic.LLAMA_8B, context=64)
    tensors = synthetic.build(cfg, seed=3)
    yield cfg, tensors
    for _, _, w in tensors.values():
        if isinstance(w, gpu.Weight):
            w.release()


def test_llama8b_shape_greedy_matches_oracle(gpu, llama8b):
    """Config 4's model at batch 1: a 32-token prompt (uniform ids, seed 7)
    and 16 greedy tokens, f16 cache (the importer's default, -kv f16); the
    GPU decoder and the CPU restatement pick the same ids on the same
    weight bytes."""
    import decoder
    import synthetic

    cfg, tensors = llama8b
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 32).astype(np.int32)
    n_new = 16
    dec = decoder.Decoder(cfg, tensors, a8=True, cache_f16=True, max_rows=32)
    got = dec.generate([prompt], n_new)[0].tolist()
    del dec
    print("llama8b GPU ids", got, flush=True)
    ref = llama_ref.Decoder(llama_ref.Model(cfg, synthetic.host_bytes(tensors)), a8=True, cache_f16=True,
                            threads=16)
    want = _oracle_greedy(ref, prompt, n_new)
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


def test_llama8b_shape_eight_slots_match_single_sequences(gpu, llama8b):
    """Config 4's batch of 8: eight distinct prompts in eight slots of one
    cache (the reference's "slots", importer/llama.go:378-395), decoded as
    one batch of rows on the matrix-core GEMV, give each prompt the ids of
    its own single-sequence run; slot 0's prompt is the batch-1 test's, whose
    ids equal the CPU restatement's."""
    import decoder

    cfg, tensors = llama8b
    rng = np.random.default_rng(7)
    prompts = np.stack([rng.integers(0, cfg["vocab"], 32) for _ in range(8)]).astype(np.int32)
    n_new = 16
    batch = decoder.Decoder(cfg, tensors, a8=True, cache_f16=True, max_rows=256, slots=8)
    got = batch.generate(prompts, n_new)
    del batch
    single = decoder.Decoder(cfg, tensors, a8=True, cache_f16=True, max_rows=32, slots=1)
    for i in range(8):
        single.reset()
        want = single.generate(prompts[i:i + 1], n_new)[0].tolist()
        assert got[i].tolist() == want, f"slot {i}"


def _cfg4_fixture():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import make_cfg4_ids

    with open(make_cfg4_ids.FIXTURE) as f:
        return make_cfg4_ids, json.load(f)


def test_llama8b_512_prompt_greedy_matches_oracle_ids(gpu, llama8b):
    """Config 4 at its stated size, batch 1: a 512-token prompt (uniform ids,
    seed 7) in one batch of 512 prompt rows, then 32 greedy tokens, f16
    cache; the GPU decoder picks the CPU restatement's ids
    (tests/golden/cfg4_ids.json, written by make_cfg4_ids.py from the same
    device-built weights, whose bytes the digests pin)."""
    import decoder
    import synthetic

    mk, fx = _cfg4_fixture()
    cfg, tensors = llama8b
    host = synthetic.host_bytes({name: tensors[name] for name in mk.DIGESTED})
    assert mk.digests(host) == fx["weights_sha256"], "the device no longer builds the fixture's weights"
    prompt = mk.prompts(cfg["vocab"])[0]
    dec = decoder.Decoder(dict(cfg, context=mk.PROMPT_LEN + mk.N_NEW), tensors, a8=True, cache_f16=True,
                          max_rows=mk.PROMPT_LEN)
    got = dec.generate([prompt], mk.N_NEW)[0].tolist()
    del dec
    print("llama8b 512-token prompt, GPU ids", got, flush=True)
    assert got == fx["ids"], next(i for i, (a, b) in enumerate(zip(got, fx["ids"])) if a != b)


def test_llama8b_eight_512_prompts_match_single_sequences(gpu, llama8b):
    """Config 4's batch of 8 at its stated size: eight distinct 512-token
    prompts in eight slots (the reference's slots, importer/llama.go:378-395),
    their 4096 prompt rows in batches of 384 (so batches straddle slots),
    then 32 greedy steps as one batch of eight rows; each slot's ids equal
    its prompt's single-sequence run (slot 0's prompt is the batch-1 test's,
    whose ids equal the CPU restatement's)."""
    import decoder

    mk, fx = _cfg4_fixture()
    cfg, tensors = llama8b
    prompts = mk.prompts(cfg["vocab"])
    c = dict(cfg, context=mk.PROMPT_LEN + mk.N_NEW)
    batch = decoder.Decoder(c, tensors, a8=True, cache_f16=True, max_rows=384, slots=mk.SLOTS)
    got = batch.generate(prompts, mk.N_NEW)
    del batch
    assert got[0].tolist() == fx["ids"]
    single = decoder.Decoder(c, tensors, a8=True, cache_f16=True, max_rows=mk.PROMPT_LEN, slots=1)
    for i in range(1, mk.SLOTS):
        single.reset()
        want = single.generate(prompts[i:i + 1], mk.N_NEW)[0].tolist()
        assert got[i].tolist() == want, f"slot {i}"


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("slots", [1, 8])
def test_attention_prompt_512_rows_bitexact(gpu, oracle, rt, f16, slots):
    """Config 4's prompt rows through attention: 512 query rows with the 8B
    heads (32 query heads, 8 kv heads, head dim 128) in a cache of 544
    entries a slot; one sequence at positions 0..511 (the causal prefill),
    or eight slots of 64 rows each; bit for bit the C restatement."""
    H, Hkv, D, T, C = 32, 8, 128, 512, 544
    rng = np.random.default_rng(512 + slots)
    L = slots * C
    cdt = np.float16 if f16 else np.float32
    kc = (rng.standard_normal((Hkv, L, D)) * 2).astype(cdt)
    vc = rng.standard_normal((Hkv, L, D)).astype(cdt)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    per = T // slots
    slot = np.arange(T) // per
    pos = (np.arange(T) % per).astype(np.int64)
    cidx = (slot * C + pos).astype(np.int64)
    kstart = (slot * C).astype(np.int64)
    dq, dk, dv, de, ds = dev(rt, q), dev(rt, kc), dev(rt, gpu.pack_vcache(vc)), dev(rt, cidx), dev(rt, kstart)
    out = rt.DeviceBuffer(q.nbytes)
    wsb = gpu.attention_workspace_bytes(T, H, C)
    ws = rt.DeviceBuffer(wsb)
    s = rt.Stream()
    gpu.attention_dev(dq.ptr, dk.ptr, dv.ptr, de.ptr, ds.ptr if slots > 1 else None, T, H, Hkv, D, L, C, f16, out.ptr,
                      ws.ptr, wsb, s.handle)
    s.sync()
    want = oracle.attention(q, kc, vc, cidx, kstart if slots > 1 else None)
    got = out.download(np.float32).reshape(T, H, D)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), float(np.max(np.abs(got - want)))


# ------------------------------------------------------ fused launches

def _ws_bytes(gpu, ws, rows, k):
    """The quantized activations in a workspace, as raw bytes per array."""
    off = gpu.a8_workspace_offsets(rows, k)
    raw = ws.download(np.uint8, gpu.a8_workspace_bytes(rows, k))
    sizes = [rows * k, rows * (k // 32) * 4, rows * (k // 32) * 2, rows * (k // 16) * 2, rows * (k // 32) * 4, rows * 4]
    return [raw[o:o + n].tobytes() for o, n in zip(off, sizes)]


@pytest.mark.parametrize("rows,n,block,resid", [(1, 4096, 256, True), (5, 2048, 256, False), (3, 1024, 32, True),
                                                (2, 8192, 256, True)])
def test_rms_norm_quant_equals_two_launches(gpu, rt, rows, n, block, resid):
    rng = np.random.default_rng(rows * n + block)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    r = rng.standard_normal((rows, n)).astype(np.float32)
    sc = rng.standard_normal(n).astype(np.float32)
    s = rt.Stream()
    wsb = gpu.a8_workspace_bytes(rows, n)
    outs = []
    for fused in (False, True):
        dx, dr, dsc, dy, ws = dev(rt, x), dev(rt, r), dev(rt, sc), rt.DeviceBuffer(x.nbytes), rt.DeviceBuffer(wsb)
        ws.zero()
        if fused:
            gpu.rms_norm_quant_dev(dx.ptr, dr.ptr if resid else None, dsc.ptr, 1e-5, rows, n, dy.ptr, block, ws.ptr, wsb,
                                   s.handle)
        else:
            gpu.rms_norm_dev(dx.ptr, dr.ptr if resid else None, dsc.ptr, 1e-5, rows, n, dy.ptr, s.handle)
            gpu.quantize_act_dev(dy.ptr, rows, n, block, ws.ptr, wsb, s.handle)
        s.sync()
        outs.append((dx.download(np.float32), dy.download(np.float32), _ws_bytes(gpu, ws, rows, n)))
    (x0, y0, q0), (x1, y1, q1) = outs
    assert np.array_equal(x0, x1)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    assert q0 == q1


_NORM_GROUPS = {
    # K, [(dtype, rows)], resid, case
    "llama8b_qkv": (4096, [(Q4_K, 512), (Q4_K, 128), (Q6_K, 128)], True, None),
    "llama1b_qkv": (2048, [(Q4_K, 2048), (Q4_K, 512), (Q6_K, 512)], False, None),
    "refused_row": (1024, [(Q6_K, 300)], True, "huge"),
    "refused_weight": (3072, [(Q4_K, 96), (Q6_K, 64)], True, "inf_scale"),
    # 768 and 512 tiles of 8 rows: three and two tiles a workgroup, one norm
    "llama8b_full_qkv": (4096, [(Q4_K, 4096), (Q4_K, 1024), (Q6_K, 1024)], True, None),
    "teams_refused_row": (4096, [(Q4_K, 4096), (Q4_K, 1024), (Q6_K, 1024)], True, "huge"),
    "teams_refused_weight": (4096, [(Q4_K, 4096)], True, "inf_scale"),
    # rows of two and three rounds of 1024: the helper teams' rounds past the
    # row are skipped (512 tiles of 16 rows, two teams; 768 of 10, three)
    "teams_k2048": (2048, [(Q4_K, 4096), (Q4_K, 2048), (Q6_K, 2048)], True, None),
    "teams_k3072": (3072, [(Q4_K, 5120), (Q4_K, 1280), (Q6_K, 1280)], True, "inf_scale"),
}


@pytest.mark.parametrize("name", sorted(_NORM_GROUPS))
def test_rms_norm_linear_group_equals_two_calls(gpu, oracle, rt, name):
    """The norm fused in front of the one-row q/k/v GEMV: x_out = x + resid
    exactly, and y bit for bit rms_norm_dev then linear_a8_group_dev (and the
    reference product of that normed row), with refused activation rows
    (an element of h above 2^60) and refused weight rows (a non-finite
    block scale) on the float32 path."""
    K, specs, resid, case = _NORM_GROUPS[name]
    rng = np.random.default_rng(K + len(specs))
    x = rng.standard_normal((1, K)).astype(np.float32)
    r = rng.standard_normal((1, K)).astype(np.float32) if resid else None
    sc = rng.standard_normal(K).astype(np.float32)
    if case == "huge":
        sc[777] = np.float32(1e30)  # |h[777]| far above 2^60: the row is refused
    wbs = []
    for i, (dt, n) in enumerate(specs):
        wb = oracle.synthetic_weight(dt, n, K, seed=40 + i)
        if case == "inf_scale" and i == 0:
            wb = bytearray(wb.tobytes())
            for row in (9, 17):  # tiles 1 and 2 of 8 rows: another team's, the next workgroup's
                o = len(wb) // n * row + 144
                wb[o:o + 2] = b"\x00\x7c"  # block 1: d = +inf
            wb = np.frombuffer(bytes(wb), np.uint8)
        wbs.append(wb)
    W = [gpu.Weight(wb, dt, n, K) for wb, (dt, n) in zip(wbs, specs)]
    if case == "inf_scale":
        assert W[0].info()[1] == 2
    bias = [rng.standard_normal(n).astype(np.float32) if i != 1 else None for i, (_, n) in enumerate(specs)]
    s = rt.Stream()
    dx, dsc = dev(rt, x), dev(rt, sc)
    dr = dev(rt, r) if resid else None
    dbs = [dev(rt, b) if b is not None else None for b in bias]
    bptrs = [b.ptr if b else 0 for b in dbs]

    xo = rt.DeviceBuffer(x.nbytes)
    ys = [rt.DeviceBuffer(n * 4) for _, n in specs]
    gpu.rms_norm_linear_a8_group_dev(W, dx.ptr, dr.ptr if dr else None, dsc.ptr, 1e-5, xo.ptr, bptrs,
                                     [y.ptr for y in ys], s.handle)
    s.sync()
    got_x = xo.download(np.float32)
    got = [y.download(np.float32) for y in ys]

    dx2, dh = dev(rt, x), rt.DeviceBuffer(x.nbytes)
    ys2 = [rt.DeviceBuffer(n * 4) for _, n in specs]
    gpu.rms_norm_dev(dx2.ptr, dr.ptr if dr else None, dsc.ptr, 1e-5, 1, K, dh.ptr, s.handle)
    gpu.linear_a8_group_dev(W, dh.ptr, 1, bptrs, 256, [y.ptr for y in ys2], None, 0, s.handle)
    s.sync()
    want_x = dx2.download(np.float32)
    h = dh.download(np.float32).reshape(1, K)
    want = [y.download(np.float32) for y in ys2]
    assert np.array_equal(got_x.view(np.uint32), want_x.view(np.uint32))
    assert np.array_equal(got_x, (x + r if resid else x).ravel())
    if case == "huge":
        assert np.abs(h).max() > 2.0 ** 60
    for i, ((dt, n), wb) in enumerate(zip(specs, wbs)):
        assert np.array_equal(got[i].view(np.uint32), want[i].view(np.uint32)), (i, np.flatnonzero(got[i] != want[i])[:5])
        ref = oracle.linear_a8(h, wb, dt, n, K, bias=bias[i], block=256).ravel()
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), i
    for w in W:
        w.release()


_ROPE_QKV = {
    # K, heads, kv heads, D, rotary, interleaved, f16 cache, context, cache index, case
    "llama8b": (4096, 32, 8, 128, 128, True, True, 40, 37, None),
    "llama1b_f32": (2048, 32, 8, 64, 64, True, False, 24, 5, None),
    "qwen2_halves_bias": (1024, 8, 2, 128, 128, False, True, 16, 15, "bias"),
    "partial_rotary": (1024, 16, 4, 64, 32, False, False, 16, 0, None),
    "refused_row": (1024, 8, 8, 128, 128, True, True, 16, 9, "huge"),
    "outside_cache": (1024, 16, 4, 64, 64, True, True, 16, 16, "outside_cache"),
}


@pytest.mark.parametrize("name", sorted(_ROPE_QKV))
def test_rms_norm_qkv_rope_kv_equals_separate_calls(gpu, oracle, rt, name):
    """The attention norm, q/k/v products, rope and the cache scatter in one
    launch at one row: q, both caches (every entry) and x_out bit for bit
    rms_norm_linear_a8_group_dev then rope_kv_dev, for llama (adjacent
    pairs) and qwen2 (halves) rotation, a partial rotary span, biases, f16
    and f32 caches, a refused activation row (float32 path) and a cache
    index outside the cache (nothing stored)."""
    K, H, Hkv, D, rot, inter, f16, C, p, case = _ROPE_QKV[name]
    rng = np.random.default_rng(K + H + D)
    x = rng.standard_normal((1, K)).astype(np.float32)
    r = rng.standard_normal((1, K)).astype(np.float32)
    sc = rng.standard_normal(K).astype(np.float32)
    if case == "huge":
        sc[101] = np.float32(1e30)
    specs = [(Q4_K, H * D), (Q4_K, Hkv * D), (Q6_K, Hkv * D)]
    W = [gpu.Weight(oracle.synthetic_weight(dt, n, K, seed=60 + i), dt, n, K) for i, (dt, n) in enumerate(specs)]
    bias = [rng.standard_normal(n).astype(np.float32) if case == "bias" else None for _, n in specs]
    dbs = [dev(rt, b) if b is not None else None for b in bias]
    bptrs = [b.ptr if b else 0 for b in dbs]
    inv = (1.0 / (10000.0 ** (np.arange(0, rot, 2, dtype=np.float64) / rot))).astype(np.float64)
    dinv = dev(rt, inv)
    dpos, dcidx = dev(rt, np.array([p + 3], np.int64)), dev(rt, np.array([p], np.int64))
    esz = 2 if f16 else 4
    kbytes, vbytes = Hkv * C * D * esz, Hkv * gpu.vcache_len(C) * D * esz
    init_k = rng.integers(0, 255, kbytes, dtype=np.uint8)
    init_v = rng.integers(0, 255, vbytes, dtype=np.uint8)
    s = rt.Stream()
    dsc, dr = dev(rt, sc), dev(rt, r)

    # fused
    dx, xo, dq = dev(rt, x), rt.DeviceBuffer(K * 4), rt.DeviceBuffer(H * D * 4)
    kc, vc = dev(rt, init_k), dev(rt, init_v)
    gpu.rms_norm_qkv_rope_kv_dev(W, dx.ptr, dr.ptr, dsc.ptr, 1e-5, xo.ptr, bptrs if case == "bias" else None, dq.ptr,
                                 dpos.ptr, dcidx.ptr, dinv.ptr, H, Hkv, D, rot, inter, C, kc.ptr, vc.ptr, f16,
                                 s.handle)
    s.sync()
    got = (xo.download(np.float32), dq.download(np.float32), kc.download(np.uint8), vc.download(np.uint8))

    # the two calls
    dx2, xo2 = dev(rt, x), rt.DeviceBuffer(K * 4)
    ys = [rt.DeviceBuffer(n * 4) for _, n in specs]
    kc2, vc2 = dev(rt, init_k), dev(rt, init_v)
    gpu.rms_norm_linear_a8_group_dev(W, dx2.ptr, dr.ptr, dsc.ptr, 1e-5, xo2.ptr, bptrs if case == "bias" else None,
                                     [y.ptr for y in ys], s.handle)
    gpu.rope_kv_dev(ys[0].ptr, ys[1].ptr, ys[2].ptr, dpos.ptr, dcidx.ptr, dinv.ptr, 1, H, Hkv, D, rot, inter, C,
                    kc2.ptr, vc2.ptr, f16, s.handle)
    s.sync()
    want = (xo2.download(np.float32), ys[0].download(np.float32), kc2.download(np.uint8), vc2.download(np.uint8))
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
    assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), np.flatnonzero(got[1] != want[1])[:8]
    assert np.array_equal(got[2], want[2])
    assert np.array_equal(got[3], want[3])
    if case == "outside_cache":
        assert np.array_equal(got[2], init_k) and np.array_equal(got[3], init_v)
    else:
        assert not np.array_equal(got[2], init_k) and not np.array_equal(got[3], init_v)
    for w in W:
        w.release()


_SWIGLU_FUSED = {
    # K, N, procs, case, rows
    "llama8b_ffn": (4096, 14336, 16, None, 1),
    "procs3_tails": (1024, 1000, 3, None, 1),  # pieces of 41 elements: f64 tails in every piece
    "procs1": (2048, 512, 1, "bias", 1),
    "refused_row": (1024, 256, 16, "huge", 1),
    "refused_weight": (1024, 512, 7, "inf_scale", 1),
    # 2..8 rows (the matrix-core GEMV's epilogue; pieces over rows * N)
    "llama8b_ffn_b8": (4096, 14336, 16, None, 8),
    "b2_procs3_tails": (1024, 1000, 3, None, 2),  # pieces of 83: tails inside rows
    "b5_procs1_bias": (2048, 512, 1, "bias", 5),
    "b8_refused_row": (1024, 256, 16, "huge", 8),
    "b4_refused_weight": (1024, 512, 7, "inf_scale", 4),
    "b3_procs7": (1024, 136, 7, None, 3),  # 17 workgroups of 8 rows
}


@pytest.mark.parametrize("name", sorted(_SWIGLU_FUSED))
def test_matmul_swiglu_equals_group_then_swiglu(gpu, oracle, rt, name):
    """gate/up products with swiglu in the epilogue: out bit for bit
    matmul_a8_quantized_group_dev then swiglu_dev (the reference's pieces for
    several GOMAXPROCS, f64 tails included), one row and 2..8 rows, with
    biases, a refused activation row and a weight row with a non-finite
    block scale (both on the float32 path)."""
    K, N, procs, case, T = _SWIGLU_FUSED[name]
    rng = np.random.default_rng(K + N + procs + T)
    x = rng.standard_normal((T, K)).astype(np.float32)
    if case == "huge":
        x[T // 2, 5] = np.float32(3e18)  # above 2^60: the row is refused
    wbs = []
    for i in range(2):
        wb = oracle.synthetic_weight(Q4_K, N, K, seed=80 + i)
        if case == "inf_scale" and i == 1:
            wb = bytearray(wb.tobytes())
            o = len(wb) // N * 9 + 2 * 144
            wb[o:o + 2] = b"\x00\x7c"  # up row 9, block 2: d = +inf
            wb = np.frombuffer(bytes(wb), np.uint8)
        wbs.append(wb)
    W = [gpu.Weight(wb, Q4_K, N, K) for wb in wbs]
    bias = [rng.standard_normal(N).astype(np.float32) for _ in range(2)] if case == "bias" else None
    dbs = [dev(rt, b) for b in bias] if bias else None
    s = rt.Stream()
    dx = dev(rt, x)
    wsb = gpu.a8_workspace_bytes(T, K)
    ws = rt.DeviceBuffer(wsb)
    gpu.quantize_act_dev(dx.ptr, T, K, 256, ws.ptr, wsb, s.handle)
    out = rt.DeviceBuffer(T * N * 4)
    gpu.matmul_a8_quantized_swiglu_dev(W, dx.ptr, T, [b.ptr for b in dbs] if dbs else None, 256, out.ptr, procs,
                                       ws.ptr, wsb, s.handle)
    g, u, want = rt.DeviceBuffer(T * N * 4), rt.DeviceBuffer(T * N * 4), rt.DeviceBuffer(T * N * 4)
    gpu.matmul_a8_quantized_group_dev(W, dx.ptr, T, [b.ptr for b in dbs] if dbs else None, 256, [g.ptr, u.ptr],
                                      ws.ptr, wsb, s.handle)
    gpu.swiglu_dev(g.ptr, u.ptr, want.ptr, T * N, procs, s.handle)
    s.sync()
    a, b = out.download(np.float32), want.download(np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))[:8]
    if case == "inf_scale":
        assert W[1].info()[1] == 1
    for w in W:
        w.release()


def test_matmul_swiglu_not_handled(gpu, oracle, rt):
    """Shapes without the swiglu epilogue are refused before any launch:
    nine rows, blocks of 32, a Q6_K weight, mismatched shapes, N a multiple
    of 4 but not of 8 at two rows."""
    s = rt.Stream()
    K = 512
    q4 = [gpu.Weight(oracle.synthetic_weight(Q4_K, 64, K, seed=9 + i), Q4_K, 64, K) for i in range(2)]
    q6 = gpu.Weight(oracle.synthetic_weight(Q6_K, 64, K, seed=11), Q6_K, 64, K)
    q4b = gpu.Weight(oracle.synthetic_weight(Q4_K, 32, K, seed=12), Q4_K, 32, K)
    q4c = [gpu.Weight(oracle.synthetic_weight(Q4_K, 36, K, seed=13 + i), Q4_K, 36, K) for i in range(2)]
    x = rt.DeviceBuffer(9 * K * 4)
    wsb = gpu.a8_workspace_bytes(9, K)
    ws, out = rt.DeviceBuffer(wsb), rt.DeviceBuffer(64 * 4 * 9)
    for ws_pair, rows, block in (((q4[0], q4[1]), 9, 256), ((q4[0], q4[1]), 1, 32), ((q4[0], q6), 1, 256),
                                 ((q4[0], q4b), 1, 256), ((q4[0], q6), 4, 256), (tuple(q4c), 2, 256)):
        with pytest.raises(gpu.NotHandled):
            gpu.matmul_a8_quantized_swiglu_dev(list(ws_pair), x.ptr, rows, None, block, out.ptr, 16, ws.ptr, wsb,
                                               s.handle)
    for w in q4 + [q6, q4b] + q4c:
        w.release()


_ROPE_QKV_ROWS = {
    # rows, K, heads, kv heads, D, rotary, interleaved, f16 cache, context, case
    "llama8b_b8": (8, 4096, 32, 8, 128, 128, True, True, 40, None),
    "llama1b_b5_f32": (5, 2048, 32, 8, 64, 64, True, False, 24, None),
    "qwen2_b4_bias": (4, 1024, 8, 2, 128, 128, False, True, 16, "bias"),
    "partial_b6": (6, 1024, 16, 4, 64, 32, False, False, 16, None),
    "refused_b8": (8, 1024, 8, 8, 128, 128, True, True, 16, "huge"),
    "q6k_qk_b7": (7, 1024, 8, 2, 64, 64, True, True, 16, "q6k"),
    "q4k_v_b8": (8, 1024, 8, 2, 128, 128, True, True, 16, "q4kv"),
}


@pytest.mark.parametrize("name", sorted(_ROPE_QKV_ROWS))
def test_qkv_rope_kv_rows_equal_separate_calls(gpu, oracle, rt, name):
    """4..8 rows: q, k, v products of quantized activations with rope and
    the cache scatter in their epilogues: q and both caches (every entry)
    bit for bit matmul_a8_quantized_group_dev then rope_kv_dev, rows in
    different slots (one cache index past the cache), adjacent-pair and
    half rotation, a partial rotary span, biases, f16/f32 caches, a refused
    activation row, Q6_K q/k and Q4_K v (one launch, q/k and v of either
    dtype)."""
    T, K, H, Hkv, D, rot, inter, f16, C, case = _ROPE_QKV_ROWS[name]
    rng = np.random.default_rng(T * K + H + D)
    x = rng.standard_normal((T, K)).astype(np.float32)
    if case == "huge":
        x[3, 17] = np.float32(5e18)
    qk_dt = Q6_K if case == "q6k" else Q4_K
    specs = [(qk_dt, H * D), (qk_dt, Hkv * D), (Q4_K if case == "q4kv" else Q6_K, Hkv * D)]
    W = [gpu.Weight(oracle.synthetic_weight(dt, n, K, seed=70 + i), dt, n, K) for i, (dt, n) in enumerate(specs)]
    bias = [rng.standard_normal(n).astype(np.float32) if case == "bias" else None for _, n in specs]
    dbs = [dev(rt, b) if b is not None else None for b in bias]
    bptrs = [b.ptr if b else 0 for b in dbs] if case == "bias" else None
    inv = (1.0 / (500000.0 ** (np.arange(0, rot, 2, dtype=np.float64) / rot))).astype(np.float64)
    dinv = dev(rt, inv)
    cidx = np.array([(t * 5 + 3) % (C + 1) for t in range(T)], np.int64)  # one index may equal C: not stored
    cidx[-1] = C
    pos = (cidx + 11).astype(np.int64)
    dpos, dcidx = dev(rt, pos), dev(rt, cidx)
    esz = 2 if f16 else 4
    kbytes, vbytes = Hkv * C * D * esz, Hkv * gpu.vcache_len(C) * D * esz
    init_k = rng.integers(0, 255, kbytes, dtype=np.uint8)
    init_v = rng.integers(0, 255, vbytes, dtype=np.uint8)
    s = rt.Stream()
    dx = dev(rt, x)
    wsb = gpu.a8_workspace_bytes(T, K)
    ws = rt.DeviceBuffer(wsb)
    gpu.quantize_act_dev(dx.ptr, T, K, 256, ws.ptr, wsb, s.handle)
    dq, kc, vc = rt.DeviceBuffer(T * H * D * 4), dev(rt, init_k), dev(rt, init_v)
    gpu.matmul_a8_quantized_qkv_rope_kv_dev(W, dx.ptr, T, bptrs, 256, dq.ptr, dpos.ptr, dcidx.ptr, dinv.ptr, H, Hkv,
                                            D, rot, inter, C, kc.ptr, vc.ptr, f16, ws.ptr, wsb, s.handle)
    ys = [rt.DeviceBuffer(T * n * 4) for _, n in specs]
    kc2, vc2 = dev(rt, init_k), dev(rt, init_v)
    gpu.matmul_a8_quantized_group_dev(W, dx.ptr, T, bptrs, 256, [y.ptr for y in ys], ws.ptr, wsb, s.handle)
    gpu.rope_kv_dev(ys[0].ptr, ys[1].ptr, ys[2].ptr, dpos.ptr, dcidx.ptr, dinv.ptr, T, H, Hkv, D, rot, inter, C,
                    kc2.ptr, vc2.ptr, f16, s.handle)
    s.sync()
    a, b = dq.download(np.float32), ys[0].download(np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))[:8]
    assert np.array_equal(kc.download(np.uint8), kc2.download(np.uint8))
    assert np.array_equal(vc.download(np.uint8), vc2.download(np.uint8))
    assert not np.array_equal(kc.download(np.uint8), init_k)
    for w in W:
        w.release()


def test_rms_norm_qkv_rope_kv_not_handled(gpu, oracle, rt):
    """Shapes the fused rope launch does not take are refused before any
    launch: q/k/v rows that are not heads*d, kv_heads*d, kv_heads*d, and a
    head whose rotation pairs would split unevenly over workgroups."""
    s = rt.Stream()
    K = 1024
    W = [gpu.Weight(oracle.synthetic_weight(Q4_K, n, K, seed=7), Q4_K, n, K) for n in (512, 128, 128)]
    dx, xo, dq = rt.DeviceBuffer(K * 4), rt.DeviceBuffer(K * 4), rt.DeviceBuffer(512 * 4)
    p = dev(rt, np.zeros(1, np.int64))
    inv = dev(rt, np.ones(32, np.float64))
    kc, vc = rt.DeviceBuffer(1 << 16), rt.DeviceBuffer(1 << 16)
    # (K = 1024: 32 rows, 16 rotation pairs, per workgroup)
    for H, Hkv, D in ((8, 2, 32), (32, 8, 16)):
        with pytest.raises(gpu.NotHandled):
            gpu.rms_norm_qkv_rope_kv_dev(W, dx.ptr, None, None, 1e-5, xo.ptr, None, dq.ptr, p.ptr, p.ptr, inv.ptr, H,
                                         Hkv, D, D, True, 8, kc.ptr, vc.ptr, True, s.handle)
    for w in W:
        w.release()


def test_rms_norm_linear_group_not_handled(gpu, oracle, rt):
    """Shapes the fused norm GEMV does not take are refused before any launch
    (NotHandled: the caller makes the two calls), and an x_out that overlaps
    x is an argument error."""
    s = rt.Stream()
    for dt, K in ((Q4_K, 1280), (Q8_0, 1024), (Q4_K, 5120)):
        w = gpu.Weight(oracle.synthetic_weight(dt, 8, K, seed=3), dt, 8, K)
        dx, xo, y = rt.DeviceBuffer(K * 4), rt.DeviceBuffer(K * 4), rt.DeviceBuffer(8 * 4)
        with pytest.raises(gpu.NotHandled):
            gpu.rms_norm_linear_a8_group_dev([w], dx.ptr, None, None, 1e-5, xo.ptr, None, [y.ptr], s.handle)
        w.release()
    w = gpu.Weight(oracle.synthetic_weight(Q4_K, 8, 1024, seed=3), Q4_K, 8, 1024)
    dx, y = rt.DeviceBuffer(2 * 1024 * 4), rt.DeviceBuffer(8 * 4)
    with pytest.raises(gpu.MimgError) as e:
        gpu.rms_norm_linear_a8_group_dev([w], dx.ptr, None, None, 1e-5, dx.ptr + 2048, None, [y.ptr], s.handle)
    assert not isinstance(e.value, gpu.NotHandled)
    w.release()


def test_swiglu_quant_out_must_be_its_own_buffer(gpu, rt):
    """swiglu_quant screens g and u for the refusal flag while it writes
    out, so an out that overlaps g or u is refused before any launch."""
    rows, n = 1, 1024
    dg, du = rt.DeviceBuffer(rows * n * 4), rt.DeviceBuffer(rows * n * 4)
    wsb = gpu.a8_workspace_bytes(rows, n)
    ws = rt.DeviceBuffer(wsb)
    s = rt.Stream()
    for out in (dg.ptr, du.ptr, dg.ptr + 2048):
        with pytest.raises(gpu.MimgError) as e:
            gpu.swiglu_quant_dev(dg.ptr, du.ptr, out, rows, n, 16, 256, ws.ptr, wsb, s.handle)
        assert not isinstance(e.value, gpu.NotHandled)


@pytest.mark.parametrize("rows,n,block,procs", [(1, 14336, 256, 16), (4, 8192, 256, 7), (3, 1792, 32, 16),
                                                (64, 14336, 256, 16)])
def test_swiglu_quant_equals_two_launches(gpu, rt, rows, n, block, procs):
    rng = np.random.default_rng(rows + n)
    g = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    u = rng.standard_normal((rows, n)).astype(np.float32)
    s = rt.Stream()
    wsb = gpu.a8_workspace_bytes(rows, n)
    outs = []
    for fused in (False, True):
        dg, du, do, ws = dev(rt, g), dev(rt, u), rt.DeviceBuffer(g.nbytes), rt.DeviceBuffer(wsb)
        ws.zero()
        if fused:
            gpu.swiglu_quant_dev(dg.ptr, du.ptr, do.ptr, rows, n, procs, block, ws.ptr, wsb, s.handle)
        else:
            gpu.swiglu_dev(dg.ptr, du.ptr, do.ptr, rows * n, procs, s.handle)
            gpu.quantize_act_dev(do.ptr, rows, n, block, ws.ptr, wsb, s.handle)
        s.sync()
        outs.append((do.download(np.float32), _ws_bytes(gpu, ws, rows, n)))
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert outs[0][1] == outs[1][1]


@pytest.mark.parametrize("block", [256, 32])
def test_swiglu_quant_refusals_match_oracle(gpu, oracle, rt, block):
    """The fused swiglu quantizer's row flags and blocks against the
    restatement (SiluMulF32 then the quantizer), with elements outside the
    quantizer's cheap screen: a huge g times a tiny u (kept), huge times huge
    (refused, |y| > 2^60), NaN (refused), in chunks past the first
    workgroup's."""
    rows, n, procs = 5, 4096, 16
    rng = np.random.default_rng(11)
    g = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    u = rng.standard_normal((rows, n)).astype(np.float32)
    g[0, 3000], u[0, 3000] = 1e10, 1e-20
    g[1, 3500], u[1, 3500] = 2.0 ** 40, 2.0 ** 30
    g[2, 4000] = np.nan
    g[3, 2100], u[3, 2100] = -1e30, 5.0
    s = rt.Stream()
    wsb = gpu.a8_workspace_bytes(rows, n)
    dg, du, do, ws = dev(rt, g), dev(rt, u), rt.DeviceBuffer(g.nbytes), rt.DeviceBuffer(wsb)
    ws.zero()
    gpu.swiglu_quant_dev(dg.ptr, du.ptr, do.ptr, rows, n, procs, block, ws.ptr, wsb, s.handle)
    s.sync()
    y = oracle.silu_mul(g.ravel(), u.ravel(), procs).reshape(rows, n)
    got_y = do.download(np.float32).reshape(rows, n)
    assert np.array_equal(got_y.view(np.uint32), y.view(np.uint32))
    q, d, xs, _, dbs, ok = _ws_bytes(gpu, ws, rows, n)
    ok = np.frombuffer(ok, np.int32)
    q = np.frombuffer(q, np.int8).reshape(rows, n)
    d = np.frombuffer(d, np.float32).reshape(rows, -1)
    for i in range(rows):
        a = oracle.Act(y[i], block)
        assert bool(ok[i]) == a.ok, i
        if a.ok:
            assert np.array_equal(q[i], a.q), i
            assert np.array_equal(d[i].view(np.uint32), np.asarray(a.d, np.float32).view(np.uint32)), i
    assert ok.tolist() == [1, 0, 0, 1, 1]


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("T,H,Hkv,D,rot,inter", [(1, 32, 8, 128, 128, True), (5, 4, 2, 64, 32, False),
                                                 (3, 8, 8, 64, 64, False), (2, 4, 1, 80, 48, True)])
def test_rope_kv_equals_three_launches(gpu, rt, f16, T, H, Hkv, D, rot, inter):
    rng = np.random.default_rng(T * D + rot)
    C = 40
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    pos = np.array([3, 17, 0, 39, 21][:T], np.int64)
    cidx = pos.copy()
    invf = np.array([500000.0 ** (-2.0 * i / rot) for i in range(rot // 2)], np.float64)
    cdt = np.float16 if f16 else np.float32
    s = rt.Stream()
    outs = []
    for fused in (False, True):
        dq, dk, dv, dp, dc, di = dev(rt, q), dev(rt, k), dev(rt, v), dev(rt, pos), dev(rt, cidx), dev(rt, invf)
        kc, vc = dev(rt, np.zeros((Hkv, C, D), cdt)), dev(rt, np.zeros((Hkv, C, D), cdt))
        if fused:
            gpu.rope_kv_dev(dq.ptr, dk.ptr, dv.ptr, dp.ptr, dc.ptr, di.ptr, T, H, Hkv, D, rot, inter, C, kc.ptr, vc.ptr,
                            f16, s.handle)
        else:
            gpu.rope_dev(dq.ptr, dp.ptr, di.ptr, T, H, D, rot, inter, s.handle)
            gpu.rope_dev(dk.ptr, dp.ptr, di.ptr, T, Hkv, D, rot, inter, s.handle)
            gpu.kv_store_dev(dk.ptr, dv.ptr, dc.ptr, T, Hkv, D, C, kc.ptr, vc.ptr, f16, s.handle)
        s.sync()
        outs.append([b.download(np.uint8).tobytes() for b in (dq, kc, vc)])
    assert outs[0] == outs[1]


def test_matmul_quantized_group_equals_single(gpu, oracle, rt):
    rows, k = 3, 1024
    specs = [(Q4_K, 300), (Q4_K, 100), (Q6_K, 120)]
    wbs = [oracle.synthetic_weight(dt, n, k, seed=40 + i) for i, (dt, n) in enumerate(specs)]
    W = [gpu.Weight(wb, dt, n, k) for wb, (dt, n) in zip(wbs, specs)]
    x = oracle.synthetic_acts(rows, k, seed=44)
    bias = np.random.default_rng(45).standard_normal(300).astype(np.float32)
    s = rt.Stream()
    wsb = gpu.a8_workspace_bytes(rows, k)
    dx, ws, db = dev(rt, x), rt.DeviceBuffer(wsb), dev(rt, bias)
    ys = [rt.DeviceBuffer(rows * n * 4) for _, n in specs]
    gpu.quantize_act_dev(dx.ptr, rows, k, 256, ws.ptr, wsb, s.handle)
    gpu.matmul_a8_quantized_group_dev(W, dx.ptr, rows, [db.ptr, None, None], 256, [y.ptr for y in ys], ws.ptr, wsb,
                                      s.handle)
    s.sync()
    for i, ((dt, n), wb) in enumerate(zip(specs, wbs)):
        want = oracle.linear_a8(x, wb, dt, n, k, bias=bias if i == 0 else None, block=256)
        got = ys[i].download(np.float32).reshape(rows, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i


@pytest.mark.parametrize("f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("T,slots,D,C", [(20, 1, 64, 64), (37, 1, 128, 64), (24, 3, 64, 64), (18, 2, 128, 64),
                                         (24, 3, 64, 44), (18, 2, 128, 42), (300, 1, 64, 320), (260, 2, 64, 140),
                                         (256, 4, 128, 70), (270, 3, 64, 100), (257, 1, 128, 300)])
def test_attention_many_queries_bitexact(gpu, oracle, rt, f16, T, slots, D, C):
    """Prompt-like batches (T >= 16 rows: four queries per workgroup; from
    256 rows a key per lane for the scores and eight queries' chains a lane
    for the weighted sum): rows of one sequence at consecutive positions (the
    causal prefill), and rows of several slots interleaved (slot starts
    inside an 8-key block of the value cache when C is not a multiple of 8;
    a workgroup's queries then see different first entries), against the C
    restatement bit for bit."""
    H, Hkv = 4, 2
    rng = np.random.default_rng(T + slots + D)
    L = slots * C
    cdt = np.float16 if f16 else np.float32
    kc = (rng.standard_normal((Hkv, L, D)) * 2).astype(cdt)
    vc = rng.standard_normal((Hkv, L, D)).astype(cdt)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    slot = np.arange(T) % slots if slots > 1 else np.zeros(T, np.int64)
    pos = np.arange(T) // slots if slots > 1 else np.arange(T)
    pos = pos.astype(np.int64) + 3
    cidx = (slot * C + pos).astype(np.int64)
    kstart = (slot * C).astype(np.int64)
    dq, dk, dv, de, ds = dev(rt, q), dev(rt, kc), dev(rt, gpu.pack_vcache(vc)), dev(rt, cidx), dev(rt, kstart)
    out = rt.DeviceBuffer(q.nbytes)
    wsb = gpu.attention_workspace_bytes(T, H, C)
    ws = rt.DeviceBuffer(wsb)
    s = rt.Stream()
    gpu.attention_dev(dq.ptr, dk.ptr, dv.ptr, de.ptr, ds.ptr if slots > 1 else None, T, H, Hkv, D, L, C, f16, out.ptr,
                      ws.ptr, wsb, s.handle)
    s.sync()
    want = oracle.attention(q, kc, vc, cidx, kstart if slots > 1 else None)
    got = out.download(np.float32).reshape(T, H, D)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), float(np.max(np.abs(got - want)))


def test_container_upload_runs_match_the_go_executor(gpu):
    """8(f)(3)/(4): the reference's importer output (a .mim container with
    its weights, metadata and graph) opened, its weights section uploaded in
    one transfer with every matrix a view at its offset, and the two runs of
    its compatibility fixture (a 7-token prompt, then one decode step at
    position 7) decoded on the GPU: every logit within 2e-5 of the largest
    of the Go executor's (the fixture's own tolerance)."""
    import binascii
    import json
    import os

    import container
    import decoder
    from conftest import GOLDEN

    exp = json.load(open(os.path.join(GOLDEN, "tiny-llama.expected.json")))
    f = container.MimFile(os.path.join(GOLDEN, "tiny-llama.mim"))
    sec, tensors = f.upload()
    dec = decoder.Decoder(f.llama_config(), tensors, a8=False, max_rows=16)

    def arr(d, dt):
        return np.frombuffer(binascii.unhexlify(d["data"]), dt)

    for run in exp["runs"]:
        toks = arr(run["inputs"]["tokens"], np.int32)
        pos = arr(run["inputs"]["positions"], np.int64)
        want = arr(run["outputs"]["logits"], np.float32)
        got = dec.forward(toks, pos).ravel()
        ok, worst, allowed = fm.near(got, want, float(run["outputs"]["logits"]["tol"]))
        assert ok, f"{worst} > {allowed}"
    del dec
    for t in list(tensors.values()):
        if isinstance(t[2], gpu.Weight):
            t[2].release()
    sec.free()
    f.close()


def _gguf_decoder(fx, **kw):
    import os

    import decoder
    import gguf
    from conftest import GOLDEN

    g = gguf.GGUFFile(os.path.join(GOLDEN, f"{fx}-tiny-q4km.gguf"))
    sec, tensors = g.upload()
    dec = decoder.Decoder(decoder.config_from_metadata(g.metadata), tensors, max_rows=16, **kw)
    return g, sec, tensors, dec


def _release(g, sec, tensors, gpu):
    for t in tensors.values():
        if isinstance(t[2], gpu.Weight):
            t[2].release()
    sec.free()
    g.close()


@pytest.mark.parametrize("name", fm.FIXTURES)
def test_gguf_model_end_to_end(gpu, name):
    """8(f)(4): the reference's GGUF fixture read by the product's GGUF
    reader, its tensor data uploaded in one transfer (views per matrix),
    the configuration from its metadata (LlamaConfigOf), and the reference's
    generate checks: f32 path within 2e-5 with the oracle's greedy ids; a8
    (dequant_matmul_a8.v2, f16 cache) within llama.cpp's deviation x1.1."""
    _, _, e = fm.load(name)
    P = len(e["prompt_ids"])
    for a8 in (False, True):
        g, sec, tensors, dec = _gguf_decoder(name, a8=a8, cache_f16=a8)
        steps = [dec.forward(e["prompt_ids"], np.arange(P))]
        for i, tok in enumerate(e["greedy"][:-1]):
            steps.append(dec.forward([tok], [P + i]))
        worst = fm.max_diff(steps[0], fm.f32b64(e["prompt_logits"]))
        for i, lg in enumerate(steps):
            last = lg[-1]
            want = fm.f32b64(e["greedy_logits"][i])
            worst = max(worst, fm.max_diff(last, want))
            if not a8:
                ok, w, allowed = fm.near(last, want, 2e-5)
                assert ok and int(np.argmax(last)) == e["greedy"][i], (i, w, allowed)
        if a8:
            assert worst <= 1.1 * e["llama_cpp_max_diff"], worst
        del dec
        _release(g, sec, tensors, gpu)


@pytest.mark.parametrize("name", fm.FIXTURES)
def test_block32_a8_graph_matches_the_restatement(gpu, name):
    """8(f)(4): dequant_matmul_a8.v1 (activation blocks of 32) for the Q4_K
    and Q6_K matrices of the fixture model, the lane order of
    dotQ4KQ8AVX2/dotQ6KQ8AVX2: the GPU decoder's logits and greedy ids
    equal the CPU restatement's with the same block."""
    cfg, tensors_np, e = fm.load(name)
    g, sec, tensors, dec = _gguf_decoder(name, a8=True, kquant_block=32)
    ref = llama_ref.Decoder(llama_ref.Model(cfg, tensors_np), a8=True, kquant_block=32, threads=4)
    P = len(e["prompt_ids"])
    a = dec.forward(e["prompt_ids"], np.arange(P))
    b = ref.forward(e["prompt_ids"], np.arange(P))
    assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(b))
    ids_g, ids_r = [], []
    lg_g, lg_r = a[-1], b[-1]
    for i in range(8):
        ids_g.append(int(np.argmax(lg_g)))
        ids_r.append(llama_ref.argmax(lg_r))
        lg_g = dec.forward([ids_g[-1]], [P + i])[0]
        lg_r = ref.forward([ids_r[-1]], [P + i])[0]
        # one-row steps too take blocks of 32 (no block-256 one-row launch)
        assert np.max(np.abs(lg_g - lg_r)) <= 1e-5 * np.max(np.abs(lg_r))
    assert ids_g == ids_r
    del dec
    _release(g, sec, tensors, gpu)
