"""Independent one-row products in one quantize launch and one product
launch (mimg_linear_a8_set_dev, and the product launch alone,
mimg_matmul_a8_quantized_set_dev) against the CPU oracle: every output bit for
bit equal, on the cfg1 layer set (an input per group), ragged and mixed
shapes up to eight groups and sixteen weights, refused input rows and weight
rows with bias, graph replays with fresh inputs, and the argument checks."""
import numpy as np
import pytest

from test_gpu_parity import Q4_K, Q6_K, Q8_0, bits_equal, first_diff

pytestmark = pytest.mark.gpu


class SetRun:
    """Device buffers of a set test: inputs, outputs and the workspace."""

    def __init__(self, gpu):
        import hiprt

        self.hiprt, self.gpu = hiprt, gpu
        self.stream = hiprt.Stream()
        self.bufs = []
        self.ws = None
        self.ws_bytes = 0

    def buf(self, nbytes):
        b = self.hiprt.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b

    def arr(self, a):
        b = self.hiprt.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))
        self.bufs.append(b)
        return b

    def workspace(self, groups):
        need = self.gpu.linear_a8_set_workspace_bytes(groups)
        if need > self.ws_bytes:
            self.ws = self.buf(need)
            self.ws_bytes = need
        return self.ws

    def enqueue(self, groups):
        ws = self.workspace(groups)
        self.gpu.linear_a8_set_dev(groups, ws.ptr, self.ws_bytes, self.stream.handle)

    def run(self, groups):
        self.enqueue(groups)
        self.stream.sync()

    def free(self):
        for b in self.bufs:
            b.free()


CFG1 = [  # (name, dtype, N, K, seed, input)
    ("q", Q4_K, 4096, 4096, 0, 0), ("k", Q4_K, 1024, 4096, 1, 0), ("v", Q6_K, 1024, 4096, 2, 0),
    ("o", Q4_K, 4096, 4096, 3, 1), ("gate", Q4_K, 14336, 4096, 4, 2), ("up", Q4_K, 14336, 4096, 5, 2),
    ("down", Q6_K, 4096, 14336, 6, 3),
]


def test_set_cfg1_layer_set(gpu, oracle):
    """The Llama-3-8B layer set at one row, four groups on independent
    inputs (q/k/v, o, gate/up, down) in one set call: equal to the oracle bit
    for bit, twice on the same workspace."""
    c = SetRun(gpu)
    ws = {}
    for name, dt, n, k, seed, _ in CFG1:
        wb = oracle.synthetic_weight(dt, n, k, seed)
        ws[name] = (wb, gpu.Weight(wb, dt, n, k))
    xs = [oracle.synthetic_acts(1, k, seed=100 + i) for i, k in enumerate([4096, 4096, 4096, 14336])]
    xd = [c.arr(x) for x in xs]
    ys = {name: c.buf(n * 4) for name, _, n, _, _, _ in CFG1}
    groups = []
    for i in range(4):
        names = [cfg[0] for cfg in CFG1 if cfg[5] == i]
        groups.append(([ws[nm][1] for nm in names], xd[i].ptr, None, [ys[nm].ptr for nm in names]))
    wants = {name: oracle.linear_a8(xs[inp], ws[name][0], dt, n, k, block=256, threads=8)[0]
             for name, dt, n, k, _, inp in CFG1}
    for rep in range(2):
        c.run(groups)
        for name in wants:
            got = ys[name].download(np.float32)
            assert bits_equal(got, wants[name]), (rep, name, first_diff(got, wants[name]))
    # the product launch alone on the rows the set call left in the
    # workspace, into fresh outputs
    ys2 = {name: c.buf(n * 4) for name, _, n, _, _, _ in CFG1}
    groups2 = [(W, xp, b, [ys2[nm].ptr for nm in [cfg[0] for cfg in CFG1 if cfg[5] == i]])
               for i, (W, xp, b, _) in enumerate(groups)]
    gpu.matmul_a8_quantized_set_dev(groups2, c.ws.ptr, c.ws_bytes, c.stream.handle)
    c.stream.sync()
    for name in wants:
        got = ys2[name].download(np.float32)
        assert bits_equal(got, wants[name]), (name, first_diff(got, wants[name]))
    for v in ws.values():
        v[1].release()
    c.free()


def test_set_mixed_shapes_eight_groups(gpu, oracle):
    """Eight groups, sixteen weights: K from 256 to 14336, N from 1 to 2051
    (tiles with a single row, rows past a tile's end), Q4_K and Q6_K in one
    group, groups of one, two and three weights."""
    specs = [  # (K, [(dtype, N, seed), ...])
        (256, [(Q4_K, 1, 1), (Q6_K, 7, 2)]),
        (14336, [(Q6_K, 301, 3), (Q4_K, 300, 4), (Q4_K, 9, 5)]),
        (2048, [(Q4_K, 2051, 6)]),
        (4096, [(Q6_K, 1024, 7), (Q4_K, 17, 8)]),
        (512, [(Q4_K, 33, 9), (Q6_K, 65, 10)]),
        (1024, [(Q6_K, 5, 11), (Q4_K, 6, 16)]),
        (7168, [(Q4_K, 130, 12), (Q6_K, 131, 13)]),
        (3072, [(Q4_K, 999, 14), (Q4_K, 1000, 15)]),
    ]
    assert sum(len(s[1]) for s in specs) == 16
    c = SetRun(gpu)
    groups, keep = [], []
    for gi, (k, mats) in enumerate(specs):
        x = oracle.synthetic_acts(1, k, seed=200 + gi)
        xd = c.arr(x)
        wbs = [(oracle.synthetic_weight(dt, n, k, seed), dt, n) for dt, n, seed in mats]
        W = [gpu.Weight(wb, dt, n, k) for wb, dt, n in wbs]
        ys = [c.buf(n * 4) for _, _, n in wbs]
        groups.append((W, xd.ptr, None, [y.ptr for y in ys]))
        keep.append((x, k, wbs, W, ys))
    c.run(groups)
    for gi, (x, k, wbs, W, ys) in enumerate(keep):
        for i, (wb, dt, n) in enumerate(wbs):
            got = ys[i].download(np.float32).reshape(1, -1)
            want = oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8)
            assert bits_equal(got, want), (gi, i, first_diff(got, want))
        for w in W:
            w.release()
    c.free()


def test_set_refusals_and_bias(gpu, oracle):
    """A NaN input row and an input above 2^60 (the whole row on the float32
    path), weight rows with an Inf or NaN block scale, and bias: equal to the
    oracle (NaN outputs where it gives NaN)."""
    k = 4096
    c = SetRun(gpu)
    wq = oracle.synthetic_weight(Q4_K, 520, k, 71).copy()
    w6 = oracle.synthetic_weight(Q6_K, 260, k, 72).copy()
    rbq, rb6 = (k // 256) * 144, (k // 256) * 210
    wq[5 * rbq + 3 * 144: 5 * rbq + 3 * 144 + 2] = np.frombuffer(np.array([0x7C00], np.uint16).tobytes(), np.uint8)
    wq[300 * rbq + 2: 300 * rbq + 4] = np.frombuffer(np.array([0x7E01], np.uint16).tobytes(), np.uint8)  # dmin NaN
    w6[17 * rb6 + 7 * 210 + 208: 17 * rb6 + 7 * 210 + 210] = np.frombuffer(np.array([0xFC00], np.uint16).tobytes(),
                                                                           np.uint8)
    Wq, W6 = gpu.Weight(wq, Q4_K, 520, k), gpu.Weight(w6, Q6_K, 260, k)
    xs = [oracle.synthetic_acts(1, k, seed=73 + i) for i in range(3)]
    xs[1][0, 1000] = np.nan
    xs[2][0, 7] = np.float32(2.0 ** 61)
    bq = np.random.default_rng(74).standard_normal(520).astype(np.float32)
    b6 = np.random.default_rng(75).standard_normal(260).astype(np.float32)
    bqd, b6d = c.arr(bq), c.arr(b6)
    xd = [c.arr(x) for x in xs]
    ys = [[c.buf(520 * 4), c.buf(260 * 4)] for _ in range(3)]
    groups = [([Wq, W6], xd[i].ptr, [bqd.ptr, b6d.ptr if i != 1 else None], [y.ptr for y in ys[i]])
              for i in range(3)]
    c.run(groups)
    for i in range(3):
        wantq = oracle.linear_a8(xs[i], wq, Q4_K, 520, k, bias=bq, block=256)
        want6 = oracle.linear_a8(xs[i], w6, Q6_K, 260, k, bias=b6 if i != 1 else None, block=256)
        gotq = ys[i][0].download(np.float32).reshape(1, -1)
        got6 = ys[i][1].download(np.float32).reshape(1, -1)
        assert bits_equal(gotq, wantq), (i, first_diff(gotq, wantq))
        assert bits_equal(got6, want6), (i, first_diff(got6, want6))
    Wq.release()
    W6.release()
    c.free()


def test_set_equals_group_calls_graph_replays(gpu, oracle):
    """A captured graph of a three-group set replayed eight times with eager
    calls between the replays and fresh inputs each time: every result equals
    the separate group calls on the same inputs, bit for bit."""
    hiprt = __import__("hiprt")
    c = SetRun(gpu)
    shapes = [(4096, [(Q4_K, 4096, 81), (Q6_K, 1024, 82)]), (14336, [(Q6_K, 2048, 83)]), (4096, [(Q4_K, 3000, 84)])]
    groups, ref_groups, xds = [], [], []
    for k, mats in shapes:
        W = [gpu.Weight(oracle.synthetic_weight(dt, n, k, seed), dt, n, k) for dt, n, seed in mats]
        xd = c.buf(k * 4)
        ys = [c.buf(n * 4) for _, n, _ in mats]
        yr = [c.buf(n * 4) for _, n, _ in mats]
        wsr = c.buf(gpu.a8_workspace_bytes(1, k))
        groups.append((W, xd.ptr, None, [y.ptr for y in ys]))
        ref_groups.append((W, xd, ys, yr, wsr, k))
        xds.append((xd, k))
    c.workspace(groups)
    g = hiprt.Graph(c.stream, lambda: c.enqueue(groups))
    for rep in range(8):
        for i, (xd, k) in enumerate(xds):
            xd.upload(oracle.synthetic_acts(1, k, seed=300 + 10 * rep + i))
        if rep % 2:
            g.launch(c.stream)
        else:
            c.enqueue(groups)
        c.stream.sync()
        for W, xd, ys, yr, wsr, k in ref_groups:
            gpu.linear_a8_group_dev(W, xd.ptr, 1, None, 256, [y.ptr for y in yr], wsr.ptr,
                                    gpu.a8_workspace_bytes(1, k), c.stream.handle)
            c.stream.sync()
            for y, r in zip(ys, yr):
                got, want = y.download(np.float32), r.download(np.float32)
                assert bits_equal(got, want), (rep, first_diff(got, want))
    for W, *_ in ref_groups:
        for w in W:
            w.release()
    c.free()


def test_set_argument_checks(gpu, oracle):
    """Overlapping outputs, an output over another group's input, a group
    without a shared K, too many groups, a Q8_0 weight (not handled) and a
    short workspace: refused before anything is launched."""
    c = SetRun(gpu)
    k = 1024
    w1 = gpu.Weight(oracle.synthetic_weight(Q4_K, 64, k, 1), Q4_K, 64, k)
    w2 = gpu.Weight(oracle.synthetic_weight(Q6_K, 64, 2048, 2), Q6_K, 64, 2048)
    w8 = gpu.Weight(oracle.synthetic_weight(Q8_0, 64, k, 3), Q8_0, 64, k)
    x = c.arr(oracle.synthetic_acts(1, k, seed=4))
    x2 = c.arr(oracle.synthetic_acts(1, k, seed=5))
    y = c.buf(64 * 4 * 2)
    good = [([w1], x.ptr, None, [y.ptr])]
    c.run(good)
    ws, wsb = c.ws, c.ws_bytes
    with pytest.raises(gpu.MimgError, match="overlap"):
        gpu.linear_a8_set_dev([([w1, w1], x.ptr, None, [y.ptr, y.ptr + 128])], ws.ptr, wsb, c.stream.handle)
    two = [([w1], x.ptr, None, [y.ptr]), ([w1], x2.ptr, None, [x.ptr])]
    ws2 = c.buf(2 * wsb)  # room for both groups, so a missed check could not write past it
    with pytest.raises(gpu.MimgError, match="overlaps the input"):
        gpu.linear_a8_set_dev(two, ws2.ptr, 2 * wsb, c.stream.handle)
    with pytest.raises(gpu.MimgError, match="share K"):
        gpu.linear_a8_set_dev([([w1, w2], x.ptr, None, [y.ptr, y.ptr + 256])], ws.ptr, wsb, c.stream.handle)
    with pytest.raises(gpu.MimgError, match="groups"):
        gpu.linear_a8_set_dev([([w1], x.ptr, None, [y.ptr])] * 9, ws.ptr, wsb, c.stream.handle)
    with pytest.raises(gpu.NotHandled):
        gpu.linear_a8_set_dev([([w8], x.ptr, None, [y.ptr])], ws.ptr, wsb, c.stream.handle)
    with pytest.raises(gpu.MimgError, match="workspace"):
        gpu.linear_a8_set_dev(good, ws.ptr, wsb - 256, c.stream.handle)
    for w in (w1, w2, w8):
        w.release()
    c.free()
