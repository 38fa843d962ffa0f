"""Host-side range check of the attention kernels' address arithmetic.

Every global and LDS address that att_scores_kernel, att_decode_kernel,
att_wsum_kernel, att_wsum_q4_kernel, att_scores_kpl_kernel and
att_wsum_qpl_kernel (mimir-model_amd/csrc/decoder_ops.hip)
compute is restated here per workgroup of the launch grid that
launch_attention picks, and its extremes are checked against the sizes of
the buffers: the key cache [kv_heads][C][D], the value cache blocked by eight
keys [kv_heads][ceil(C/8)][D][8], q and out [T][H][D], the workspace
[T][H][max_keys], and each kernel's LDS. The visible ranges come from
adversarial end/start indices (negative, past C, past max_keys, empty
ranges), over D = 8..512, one to many queries, slots, max_keys up to the
8192 limit. CPU only: nothing here runs a kernel."""
import itertools

import numpy as np
import pytest

LDS_BYTES = 160 * 1024
ATT_DEC_MAXK = 256


def att_range(kend, kstart, t, C, maxk):
    k0 = 0 if kstart is None else min(max(int(kstart[t]), 0), C - 1)
    n = int(kend[t]) + 1 - k0
    n = min(n, C - k0, maxk)
    return k0, max(n, 0)


class Bounds:
    def __init__(self, T, H, Hkv, D, C, maxk, f16):
        self.T, self.H, self.Hkv, self.D, self.C, self.maxk, self.f16 = T, H, Hkv, D, C, maxk, f16
        self.esz = 2 if f16 else 4
        self.kc_len = Hkv * C * D
        self.vc_len = Hkv * ((C + 7) // 8) * 8 * D
        self.ws_len = T * H * maxk

    def vcache_at(self, hk, j, d):
        return ((hk * ((self.C + 7) // 8) + j // 8) * self.D + d) * 8 + j % 8

    def check(self, lo, hi, size, what):
        assert 0 <= lo and hi < size, f"{what}: [{lo}, {hi}] outside [0, {size})"


def check_scores(b, ranges, QT):
    D, C = b.D, b.C
    tiles = (b.maxk + 63) // 64
    for z in range((b.T + QT - 1) // QT):
        r = [ranges[QT * z + i] if QT * z + i < b.T else (0, 0) for i in range(QT)]
        nmax = max(n for _, n in r)
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            for tile in range(tiles):
                if tile * 64 >= nmax:
                    continue
                i0 = next(i for i in range(QT) if r[i][1] > 0)
                same = all(n == 0 or k0 == r[i0][0] for k0, n in r)
                loads = [(hk * C + r[i0][0], nmax)] if same else \
                    [(hk * C + k0, n) for k0, n in r if tile * 64 < n]
                for base, nlim in loads:
                    js = (tile * 64, tile * 64 + 63)  # j0 = tile*64 + grp, j1 = j0 + 32
                    a_lo = base + min(js[0], nlim - 1)
                    a_hi = base + min(js[1], nlim - 1)
                    assert a_lo >= hk * C
                    b.check(a_lo * D, a_hi * D + D - 1, b.kc_len, "scores: key element")
                for i, (_, n) in enumerate(r):
                    if tile * 64 < n:
                        t = QT * z + i
                        b.check((t * b.H + h) * D, (t * b.H + h) * D + D - 1, b.T * b.H * D, "scores: q")
                        jw = min(tile * 64 + 63, n - 1)
                        assert jw < b.maxk
                        b.check((t * b.H + h) * b.maxk, (t * b.H + h) * b.maxk + jw, b.ws_len, "scores: out")


def check_decode(b, ranges):
    D, C, DG = b.D, b.C, 32
    PPB, VPAD = (1, 8) if b.f16 else (2, 4)
    mk = (b.maxk + 3) & ~3
    vstride = ((b.maxk + 14) & ~7) + VPAD
    lds = mk * 4 + DG * vstride * b.esz
    assert lds <= LDS_BYTES - 64
    for t, (k0, n) in enumerate(ranges):
        if n <= 0:
            continue
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            base = hk * C + k0
            # keys j + 64, j + 96 past n: the last key
            b.check(base * D, (base + n - 1) * D + D - 1, b.kc_len, "decode: key element")
            assert n <= mk  # scores sc[j], j < n
            k0a, off = k0 & ~7, k0 - (k0 & ~7)
            nblk = (off + n + 7) >> 3
            for d0 in range(0, D, DG):
                src = b.vcache_at(hk, k0a, d0)
                last = src + ((nblk - 1) * D + DG - 1) * 8 + (PPB - 1) * 4 + 16 // b.esz - 1
                b.check(src, last, b.vc_len, "decode: value element")
                # LDS dim rows: writes up to 8*nblk, chain reads up to off + n
                assert 8 * nblk <= vstride and off + n <= vstride
                assert (DG - 1) * vstride + 8 * nblk <= DG * vstride


def check_wsum(b, ranges):
    D, C = b.D, b.C
    PPB, BB, NR = (1, 16, 4) if b.f16 else (2, 16, 3)
    CPB = BB // 2 if b.f16 else BB  # copies a batch a copying wave (waves 1 and 2)
    batch = BB * PPB * 1024
    e_len = (b.maxk + 14) & ~7
    assert NR * batch + e_len * 4 + 64 <= LDS_BYTES
    assert 16 * 63 + 16 + ((BB - 1) * PPB + PPB - 1) * 1024 <= batch  # a lane's slot reads and copies
    for t, (k0, n) in enumerate(ranges):
        if n <= 0:
            continue
        k0a, off = k0 & ~7, k0 - (k0 & ~7)
        nb = (off + n + 7) >> 3
        nv = n & ~7 if n >= 8 else 0
        assert off + n - 1 < e_len  # e[off + j]; the exps' clamped reads e[off + min(j, nv - 1)], e[off + nv + tid]
        for bt in range((nb + BB - 1) // BB):  # a whole batch's chain reads e[8*b0 .. 8*(b0+BB)) only when inside
            b0 = BB * bt
            if 8 * b0 >= off and 8 * (b0 + BB) <= off + n:
                assert 8 * (b0 + BB) <= e_len
        # copies: NR - 1 batches ahead of batch 0 and one a batch after, blocks past nb: the last again
        assert (NR - 1) * CPB <= 63  # copies in flight a copying wave (vmcnt)
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            for d0 in range(0, D, 64):
                for lane in (0, 63):
                    d = min(d0 + lane, D - 1)
                    for w1 in range(PPB):
                        src = b.vcache_at(hk, k0a, d) + 4 * w1
                        last = src + (nb - 1) * 8 * D + 16 // b.esz - 1  # blocks past nb: the last again
                        b.check(src, last, b.vc_len, "wsum: value element")
                # scores: loads of j and, past the end, the last key (j clamped to n - 1)
                b.check((t * b.H + h) * b.maxk, (t * b.H + h) * b.maxk + n - 1, b.ws_len, "wsum: scores")


def check_wsum_q4(b, ranges):
    D, C = b.D, b.C
    VC, VS = (128, 136) if b.f16 else (64, 76)
    PPB = 1 if b.f16 else 2
    mkp = (b.maxk + 3) & ~3
    assert 4 * mkp * 4 + VS * 64 * b.esz <= LDS_BYTES
    for z in range((b.T + 3) // 4):
        r = [ranges[4 * z + i] if 4 * z + i < b.T else (0, 0) for i in range(4)]
        ns = [n for _, n in r]
        nmax = max(ns)
        first = next((i for i in range(4) if ns[i] > 0), -1)
        same = all(n == 0 or k0 == r[first if first >= 0 else 0][0] for k0, n in r)
        for n in ns:
            assert n <= mkp
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            for pas in range(1 if same else 4):
                src = (first if first >= 0 else 0) if same else pas
                pn = nmax if same else ns[pas]
                for c0 in range(0, pn, VC):
                    rows = min(pn - c0, VC)
                    ka = r[src][0] + c0
                    kaa, offc = ka & ~7, ka - (ka & ~7)
                    nblk = (offc + rows + 7) >> 3
                    for d0 in range(0, D, 64):
                        s0 = b.vcache_at(hk, kaa, d0)
                        last = s0 + ((nblk - 1) * D + 63) * 8 + (PPB - 1) * 4 + 16 // b.esz - 1
                        b.check(s0, last, b.vc_len, "wsum_q4: value element")
                    assert 8 * nblk <= VS and offc + rows <= VS


def check_scores_kpl(b, ranges):
    """att_scores_kpl_kernel: workgroup (x, h, z) walks tiles of 256 cache
    entries from the smallest first entry of its 32 queries, gridDim.x
    apart; thread i reads key kb + i (clamped to the cache), stores the
    score of key j = kb + i - k0 for 0 <= j < n."""
    D, C, QG = b.D, b.C, 32
    assert QG * D * 4 <= 64 * 1024  # the query rows in LDS
    gx = (b.maxk + 255) // 256
    for z in range((b.T + QG - 1) // QG):
        r = [ranges[QG * z + i] if QG * z + i < b.T else (0, 0) for i in range(QG)]
        live = [(k0, n) for k0, n in r if n > 0]
        if not live:
            continue
        kmin = min(k0 for k0, _ in live)
        kfin = max(k0 + n for k0, n in live)
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            for x in range(gx):
                kb = kmin + 256 * x
                while kb < kfin:
                    a_lo, a_hi = min(kb, C - 1), min(kb + 255, C - 1)
                    b.check((hk * C + a_lo) * D, (hk * C + a_hi) * D + D - 1, b.kc_len, "scores_kpl: key element")
                    for i, (k0, n) in enumerate(r):
                        if n <= 0:
                            continue
                        j_lo, j_hi = max(kb - k0, 0), min(kb + 255 - k0, n - 1)
                        if j_lo > j_hi:
                            continue
                        t = QG * z + i
                        assert t < b.T and j_hi < b.maxk
                        b.check((t * b.H + h) * b.maxk + j_lo, (t * b.H + h) * b.maxk + j_hi, b.ws_len,
                                "scores_kpl: out")
                    kb += 256 * gx


def check_wsum_qpl(b, ranges):
    """att_wsum_qpl_kernel: workgroup (h, z) of 16 queries; the scores of
    each query (j < n) into LDS [key][16]; per pass (all queries when they
    share the first entry, else one query at a time) the value blocks from
    the block holding k0, four ahead and clamped to the last block, and the
    LDS rows of keys below the pass's largest count."""
    D, C, QG = b.D, b.C, 16
    assert b.maxk * QG * 4 + 1024 <= LDS_BYTES
    for z in range((b.T + QG - 1) // QG):
        r = [ranges[QG * z + i] if QG * z + i < b.T else (0, 0) for i in range(QG)]
        ns = [n for _, n in r]
        for i, n in enumerate(ns):
            assert n <= b.maxk
            if n > 0:
                assert QG * z + i < b.T
        live = [i for i in range(QG) if ns[i] > 0]
        if not live:
            continue
        same = all(r[i][0] == r[live[0]][0] for i in live)
        passes = [live] if same else [[i] for i in live]
        for h in range(b.H):
            hk = h // (b.H // b.Hkv)
            for qs in passes:
                k0 = r[qs[0]][0]
                nmax = max(ns[i] for i in qs)
                off = k0 & 7
                kbeg = k0 - off
                nblk = (off + nmax + 7) >> 3
                last_blk = kbeg + 8 * (nblk - 1)
                assert kbeg >= 0 and last_blk < ((C + 7) // 8) * 8
                for d in (0, D - 1):
                    b.check(b.vcache_at(hk, kbeg, d), b.vcache_at(hk, last_blk, d) + 7, b.vc_len,
                            "wsum_qpl: value element")
                assert nmax - 1 < b.maxk  # LDS rows of the keys read


def run_launch(T, H, Hkv, D, C, maxk, f16, kend, kstart):
    b = Bounds(T, H, Hkv, D, C, maxk, f16)
    ranges = [att_range(kend, kstart, t, C, maxk) for t in range(T)]
    for k0, n in ranges:
        assert 0 <= k0 < C and 0 <= n <= min(C - k0, maxk)
    many = T >= 16 and D % 64 == 0 and maxk <= 2048
    if many and T >= 256 and (D == 64 or (D == 128 and f16)) and maxk <= 1024:
        check_scores_kpl(b, ranges)
        check_wsum_qpl(b, ranges)
        return "prompt"
    if many:
        check_scores(b, ranges, 4)
        check_wsum_q4(b, ranges)
        return "many"
    if D in (64, 128) and maxk <= ATT_DEC_MAXK:
        check_decode(b, ranges)
        return "decode"
    # (att_scores_gqa_kernel, taken for D 64/128 and 2/4/8 query heads per
    # kv head, reads the same key rows per tile and writes the same score
    # rows as the per-head kernel checked here)
    check_scores(b, ranges, 1)
    check_wsum(b, ranges)
    return "two"


def ranges_for(T, C, maxk, slots, rng):
    """End/start indices of T queries in `slots` slots of C entries, with
    adversarial values mixed in: negative, past C, empty, past max_keys."""
    L = C // slots
    kend = np.empty(T, np.int64)
    kstart = np.empty(T, np.int64)
    for t in range(T):
        s = t % slots
        kstart[t] = s * L
        kend[t] = s * L + rng.integers(0, L)
    special = [(-5, -1), (C + 9, C + 3), (C - 1, C - 1), (0, C - 1), (C - 1, 0), (7, 3), (maxk + 50, 0),
               (C * 2, -7), (C - 1, C - 9)]
    for t in range(min(T, len(special))):
        kend[t], kstart[t] = special[t]
    return kend, kstart


@pytest.mark.parametrize("D", [8, 32, 64, 96, 128, 256, 512])
@pytest.mark.parametrize("f16", [True, False])
def test_attention_addresses_in_bounds(D, f16):
    rng = np.random.default_rng(D + (1000 if f16 else 0))
    seen = set()
    for T, (H, Hkv), C, slots, maxk_kind in itertools.product(
            (1, 3, 8, 16, 37, 300), ((4, 1), (8, 2), (4, 4)), (1, 7, 42, 301, 2048, 8200), (1, 3),
            ("C", "small", "max")):
        if slots > C:
            continue
        maxk = {"C": min(C, 8192), "small": max(1, min(C, 8192) // 3), "max": 8192}[maxk_kind]
        if T * maxk > 8 * 8192 * 37:
            continue
        kend, kstart = ranges_for(T, C, maxk, slots, rng)
        seen.add(run_launch(T, H, Hkv, D, C, maxk, f16, kend, kstart if slots > 1 or T > 5 else None))
    if D == 64 or (D == 128 and f16):
        assert seen == {"many", "decode", "two", "prompt"}
    elif D == 128:
        assert seen == {"many", "decode", "two"}
    elif D % 64 == 0:
        assert seen == {"many", "two"}
