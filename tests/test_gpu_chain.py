"""The one-launch chain of one-row products (mimg_linear_a8_chain_dev)
against the CPU oracle and the separate calls: every output bit for bit
equal, for independent inputs (the cfg1 layer set), for phases that read
earlier phases' outputs, ragged and tiny shapes (workgroups with no rows in
a phase), refused input rows and weight rows, bias, repeated launches and
graph replays of one sync buffer."""
import numpy as np
import pytest

from test_gpu_parity import Q4_K, Q6_K, Q8_0, bits_equal, first_diff

pytestmark = pytest.mark.gpu


class Chain:
    """Device buffers of a chain test: inputs, outputs and a sync buffer."""

    def __init__(self, gpu):
        import hiprt

        self.hiprt, self.gpu = hiprt, gpu
        self.stream = hiprt.Stream()
        self.bufs = []
        self.sync_bytes = gpu.chain_sync_bytes()
        self.sync = self.buf(self.sync_bytes)
        gpu.chain_sync_init(self.sync.ptr, self.sync_bytes, self.stream.handle)

    def buf(self, nbytes):
        b = self.hiprt.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b

    def arr(self, a):
        b = self.hiprt.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))
        self.bufs.append(b)
        return b

    def run(self, phases):
        self.gpu.linear_a8_chain_dev(phases, self.sync.ptr, self.sync_bytes, self.stream.handle)
        self.stream.sync()

    def status(self):
        return self.gpu.chain_status(self.sync.ptr)

    def free(self):
        for b in self.bufs:
            b.free()


def _mats(gpu, oracle, specs, k):
    wbs = [oracle.synthetic_weight(dt, n, k, seed) for dt, n, seed in specs]
    return wbs, [gpu.Weight(wb, dt, n, k) for wb, (dt, n, _) in zip(wbs, specs)]


CFG1 = [  # (name, dtype, N, K, seed, input)
    ("q", Q4_K, 4096, 4096, 0, 0), ("k", Q4_K, 1024, 4096, 1, 0), ("v", Q6_K, 1024, 4096, 2, 0),
    ("o", Q4_K, 4096, 4096, 3, 1), ("gate", Q4_K, 14336, 4096, 4, 2), ("up", Q4_K, 14336, 4096, 5, 2),
    ("down", Q6_K, 4096, 14336, 6, 3),
]


def test_chain_cfg1_layer_set(gpu, oracle):
    """The Llama-3-8B layer set at one row as four phases (q/k/v, o,
    gate/up, down) on independent inputs: equal to the oracle, bit for bit,
    and to the group calls; a second launch on the same sync buffer too."""
    c = Chain(gpu)
    ws = {}
    for name, dt, n, k, seed, _ in CFG1:
        wb = oracle.synthetic_weight(dt, n, k, seed)
        ws[name] = (wb, gpu.Weight(wb, dt, n, k), dt, n, k)
    xs = [oracle.synthetic_acts(1, k, seed=100 + i) for i, k in enumerate([4096, 4096, 4096, 14336])]
    xd = [c.arr(x) for x in xs]
    ys = {name: c.buf(n * 4) for name, _, n, _, _, _ in CFG1}
    phases = []
    for i in range(4):
        names = [cfg[0] for cfg in CFG1 if cfg[5] == i]
        phases.append(([ws[nm][1] for nm in names], xd[i].ptr, None, [ys[nm].ptr for nm in names]))
    for rep in range(2):
        c.run(phases)
        assert c.status() == 0
        for name, dt, n, k, _, inp in CFG1:
            got = ys[name].download(np.float32)
            want = oracle.linear_a8(xs[inp], ws[name][0], dt, n, k, block=256, threads=8)[0]
            assert bits_equal(got, want), (rep, name, first_diff(got, want))
    for v in ws.values():
        v[1].release()
    c.free()


@pytest.mark.parametrize("case", ["llama8b_ffn", "mixed_small"])
def test_chain_dependent_phases(gpu, oracle, case):
    """Each phase reads the row the previous phase wrote (o -> gate/up; up's
    output -> down; the down output -> q/k/v), as a decoder layer's linears
    feed each other: equal to the oracle applied in turn."""
    if case == "llama8b_ffn":
        k0, specs = 4096, [[(Q4_K, 4096, 41)], [(Q4_K, 14336, 42), (Q4_K, 14336, 43)], [(Q6_K, 4096, 44)],
                           [(Q4_K, 4096, 45), (Q4_K, 1024, 46), (Q6_K, 1024, 47)]]
        feeds = [None, (0, 0), (1, 1), (2, 0)]  # (phase, output) that is this phase's input
    else:
        # 2048 -> (2048 Q6_K, 301 Q4_K) -> 256 -> (7, 9): the last phase has
        # 16 rows, so most workgroups have no rows in it
        k0, specs = 2048, [[(Q6_K, 2048, 51), (Q4_K, 301, 52)], [(Q4_K, 256, 53)], [(Q4_K, 7, 54), (Q4_K, 9, 55)]]
        feeds = [None, (0, 0), (1, 0)]
    c = Chain(gpu)
    x0 = oracle.synthetic_acts(1, k0, seed=60)
    mats, ys, phases, inputs_host = [], [], [], []
    for p, sp in enumerate(specs):
        if feeds[p] is None:
            k, xh = k0, x0
            xdev = c.arr(xh)
        else:
            fp, fo = feeds[p]
            k = specs[fp][fo][1]
            xh, xdev = None, ys[fp][fo]
        wb_w = [(oracle.synthetic_weight(dt, n, k, seed), dt, n) for dt, n, seed in sp]
        W = [gpu.Weight(wb, dt, n, k) for wb, dt, n in wb_w]
        yb = [c.buf(n * 4) for _, _, n in wb_w]
        mats.append((wb_w, W, k))
        ys.append(yb)
        inputs_host.append(xh)
        phases.append((W, xdev.ptr, None, [y.ptr for y in yb]))
    c.run(phases)
    assert c.status() == 0
    outs = []
    for p, (wb_w, W, k) in enumerate(mats):
        x = inputs_host[p] if feeds[p] is None else outs[feeds[p][0]][feeds[p][1]]
        want = [oracle.linear_a8(x, wb, dt, n, k, block=256, threads=8) for wb, dt, n in wb_w]
        outs.append(want)
        for i, y in enumerate(ys[p]):
            got = y.download(np.float32).reshape(1, -1)
            assert bits_equal(got, want[i]), (p, i, first_diff(got, want[i]))
        for w in W:
            w.release()
    c.free()


def test_chain_refusals_and_bias(gpu, oracle):
    """A NaN input row and an input above 2^60 (the whole row on the float32
    path), weight rows with an Inf or NaN block scale, and bias: equal to the
    oracle (NaN outputs where it gives NaN)."""
    k = 4096
    c = Chain(gpu)
    wq = oracle.synthetic_weight(Q4_K, 520, k, 71)
    w6 = oracle.synthetic_weight(Q6_K, 260, k, 72)
    wq = wq.copy()
    w6 = w6.copy()
    rbq, rb6 = (k // 256) * 144, (k // 256) * 210
    wq[5 * rbq + 3 * 144: 5 * rbq + 3 * 144 + 2] = np.frombuffer(np.array([0x7C00], np.uint16).tobytes(), np.uint8)
    wq[300 * rbq + 2: 300 * rbq + 4] = np.frombuffer(np.array([0x7E01], np.uint16).tobytes(), np.uint8)  # dmin NaN
    w6[17 * rb6 + 7 * 210 + 208: 17 * rb6 + 7 * 210 + 210] = np.frombuffer(np.array([0xFC00], np.uint16).tobytes(), np.uint8)
    Wq, W6 = gpu.Weight(wq, Q4_K, 520, k), gpu.Weight(w6, Q6_K, 260, k)
    xs = [oracle.synthetic_acts(1, k, seed=73 + i) for i in range(3)]
    xs[1][0, 1000] = np.nan
    xs[2][0, 7] = np.float32(2.0 ** 61)
    bq = np.random.default_rng(74).standard_normal(520).astype(np.float32)
    b6 = np.random.default_rng(75).standard_normal(260).astype(np.float32)
    bqd, b6d = c.arr(bq), c.arr(b6)
    xd = [c.arr(x) for x in xs]
    ys = [[c.buf(520 * 4), c.buf(260 * 4)] for _ in range(3)]
    phases = [([Wq, W6], xd[i].ptr, [bqd.ptr, b6d.ptr if i != 1 else None], [y.ptr for y in ys[i]]) for i in range(3)]
    c.run(phases)
    assert c.status() == 0
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


def test_chain_graph_replays(gpu, oracle):
    """A captured graph of a dependent three-phase chain replayed eight times
    with eager launches of the same chain between replays and a fresh input
    each time: every replay equals the oracle, the status stays clear."""
    hiprt = __import__("hiprt")
    k = 4096
    c = Chain(gpu)
    w0 = oracle.synthetic_weight(Q4_K, 4096, k, 81)
    w1 = oracle.synthetic_weight(Q6_K, 2048, k, 82)
    w2 = oracle.synthetic_weight(Q4_K, 512, 2048, 83)
    W0, W1, W2 = gpu.Weight(w0, Q4_K, 4096, k), gpu.Weight(w1, Q6_K, 2048, k), gpu.Weight(w2, Q4_K, 512, 2048)
    xd = c.buf(k * 4)
    y0, y1, y2 = c.buf(4096 * 4), c.buf(2048 * 4), c.buf(512 * 4)
    phases = [([W0], xd.ptr, None, [y0.ptr]), ([W1], y0.ptr, None, [y1.ptr]), ([W2], y1.ptr, None, [y2.ptr])]
    g = hiprt.Graph(c.stream, lambda: gpu.linear_a8_chain_dev(phases, c.sync.ptr, c.sync_bytes, c.stream.handle))
    for rep in range(8):
        x = oracle.synthetic_acts(1, k, seed=90 + rep)
        xd.upload(x)
        if rep % 2:
            g.launch(c.stream)
        else:
            gpu.linear_a8_chain_dev(phases, c.sync.ptr, c.sync_bytes, c.stream.handle)
        c.stream.sync()
        a = oracle.linear_a8(x, w0, Q4_K, 4096, k, block=256, threads=8)
        b = oracle.linear_a8(a, w1, Q6_K, 2048, k, block=256, threads=8)
        want = oracle.linear_a8(b, w2, Q4_K, 512, 2048, block=256, threads=8)
        got = y2.download(np.float32).reshape(1, -1)
        assert bits_equal(got, want), (rep, first_diff(got, want))
    assert c.status() == 0
    g.destroy()
    for w in (W0, W1, W2):
        w.release()
    c.free()


def test_chain_refuses_what_it_cannot_run(gpu, oracle):
    """Q8_0 weights and Q6_K rows that are not a multiple of 16 bytes are not
    handled (nothing launched); an output over its phase's input, outputs
    that overlap each other and a short sync buffer are argument errors."""
    c = Chain(gpu)
    x = c.arr(oracle.synthetic_acts(1, 4096, seed=1))
    y = c.buf(4096 * 4)
    w8 = gpu.Weight(oracle.synthetic_weight(Q8_0, 64, 4096, 1), Q8_0, 64, 4096)
    w6 = gpu.Weight(oracle.synthetic_weight(Q6_K, 64, 1024, 2), Q6_K, 64, 1024)  # 840-byte rows
    wq = gpu.Weight(oracle.synthetic_weight(Q4_K, 64, 4096, 3), Q4_K, 64, 4096)
    with pytest.raises(gpu.NotHandled):
        c.run([([w8], x.ptr, None, [y.ptr])])
    with pytest.raises(gpu.NotHandled):
        c.run([([w6], y.ptr, None, [x.ptr])])
    with pytest.raises(gpu.MimgError):
        c.run([([wq], x.ptr, None, [x.ptr + 64])])
    with pytest.raises(gpu.MimgError):
        c.run([([wq, wq], x.ptr, None, [y.ptr, y.ptr + 128])])
    with pytest.raises(gpu.MimgError):
        gpu.linear_a8_chain_dev([([wq], x.ptr, None, [y.ptr])], c.sync.ptr, 64, c.stream.handle)
    for w in (w8, w6, wq):
        w.release()
    c.free()
