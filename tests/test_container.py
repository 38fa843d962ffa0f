"""The mim container reader (mimir-model_amd/container.py) against the
reference's compatibility fixture (testdata/compat/0.2-0.1/tiny-llama.mim
and its expected.json: container version, sections, tensor table with a
SHA-256 per tensor, metadata) and the hostile corpus of spec/container.md
section 9.1, derived here from the valid file one fault at a time (the
reference derives its own in hostile_test.go)."""
import hashlib
import json
import os
import struct

import pytest

import container
from conftest import GOLDEN

MIM = os.path.join(GOLDEN, "tiny-llama.mim")
EXPECTED = json.load(open(os.path.join(GOLDEN, "tiny-llama.expected.json")))


@pytest.fixture(scope="module")
def mim():
    f = container.MimFile(MIM)
    yield f
    f.close()


def test_preamble_and_sections(mim):
    c = EXPECTED["container"]
    assert (mim.major, mim.minor, mim.data_alignment) == (c["major"], c["minor"], c["data_alignment"])
    got = sorted((k, v[1], v[2]) for k, v in mim.sections.items())
    want = sorted((s["kind"], s["length"], s["hash_algorithm"]) for s in EXPECTED["sections"])
    assert got == want
    mim.verify_hashes()


def test_tensor_table_and_bytes(mim):
    want = EXPECTED["tensors"]
    assert [t.name for t in mim.tensors] == [t["name"] for t in want]
    for t, w in zip(mim.tensors, want):
        assert container.DTYPES[t.dtype][0] == w["dtype"], t.name
        assert t.shape == w["shape"] and t.offset == w["offset"], t.name
        assert hashlib.sha256(mim.tensor_bytes(t.name)).hexdigest() == w["sha256"], t.name


def test_metadata(mim):
    m = mim.metadata()
    for e in EXPECTED["metadata"]:
        v = m[e["key"]]
        if e["type"] == "float":
            assert struct.pack("<d", v).hex() == e["value"], e["key"]
        elif e["type"] == "floats":
            assert [struct.pack("<d", x).hex() for x in v] == e["value"], e["key"]
        else:
            assert v == e["value"], e["key"]
    cfg = mim.llama_config()
    assert (cfg["layers"], cfg["embed"], cfg["heads"], cfg["kv_heads"], cfg["context"]) == (2, 256, 4, 2, 64)


# --------------------------------------------------------- hostile corpus

RAW = open(MIM, "rb").read()


def _u(fmt, off, val, b):
    b = bytearray(b)
    struct.pack_into("<" + fmt, b, off, val)
    return bytes(b)


def _layout(b):
    ioff, ilen = struct.unpack_from("<QQ", b, 16)
    ns, nt, pool = struct.unpack_from("<IIQ", b, ioff)
    sec0 = ioff + 16
    ten0 = sec0 + 64 * ns
    return ioff, ilen, ns, nt, pool, sec0, ten0


def _section(b, kind):
    _, _, ns, _, _, sec0, _ = _layout(b)
    for i in range(ns):
        if struct.unpack_from("<I", b, sec0 + 64 * i)[0] == kind:
            return sec0 + 64 * i
    raise KeyError(kind)


def _tensor_entries(b):
    _, _, _, nt, _, _, ten0 = _layout(b)
    out = []
    for i in range(nt):
        p = ten0 + 96 * i
        dt, rank = struct.unpack_from("<IB", b, p + 8)
        dims = struct.unpack_from("<8Q", b, p + 16)[:rank]
        off, ln = struct.unpack_from("<QQ", b, p + 80)
        out.append((p, dt, dims, off, ln))
    return out


def hostile():
    b = RAW
    ioff, ilen, ns, nt, pool, sec0, ten0 = _layout(b)
    ents = _tensor_entries(b)
    by_off = sorted(ents, key=lambda e: (e[3], e[4]))
    dlen = struct.unpack_from("<Q", b, 40)[0]
    small = next(e for e in by_off if e[3] > 0 and e[4] < (1 << 20))
    last = by_off[-1]
    cases = {
        "truncated-preamble": (b[:32], "truncated"),
        "bad-magic": (b"X" + b[1:], "bad-magic"),
        "big-endian": (_u("I", 8, 0x0D0C0B0A, b), "big-endian"),
        "major-version": (_u("H", 4, 1, b), "unsupported-version"),
        "reserved-preamble": (_u("Q", 56, 1, b), "reserved-non-zero"),
        "alignment-not-pow2": (_u("I", 12, 12288, b), "bad-alignment"),
        "truncated-file": (b[:-1], "truncated"),
        "trailing-bytes": (b + b"\0", "bad-length"),
        "index-too-large": (_u("Q", 24, (256 << 20) + 8, b), "index-too-large"),
        "index-out-of-bounds": (_u("Q", 24, len(b), b), "out-of-bounds"),
        "index-length-mismatch": (_u("Q", 24, ilen + 8, b), "bad-length"),
        "weights-disagree": (_u("Q", _section(b, 1) + 16, dlen - 64, b), "bad-length"),
        "unknown-required-section": (_u("I", _section(b, 2) + 4, 1, _u("I", _section(b, 2), 9, b)),
                                     "unknown-required-section"),
        "bad-hash-alg": (_u("B", _section(b, 2) + 24, 2, b), "bad-hash-algorithm"),
        "section-flags": (_u("I", _section(b, 2) + 4, 2, b), "reserved-non-zero"),
        "name-out-of-pool": (_u("I", ten0, pool + 1, b), "out-of-bounds"),
        "unsorted-names": (b[:ten0] + b[ten0 + 96:ten0 + 192] + b[ten0:ten0 + 96] + b[ten0 + 192:], "unsorted"),
        "bad-dtype": (_u("I", ten0 + 8, 999, b), "bad-dtype"),
        "rank-too-big": (_u("B", ten0 + 12, 9, b), "bad-shape"),
        "size-mismatch": (_u("Q", ten0 + 88, ents[0][4] + 1, b), "size-mismatch"),
        "shape-overflow": (_u("Q", ten0 + 16, 1 << 40, _u("Q", ten0 + 24, 1 << 40, b)), "overflow"),
        "misaligned-tensor": (_u("Q", small[0] + 80, small[3] + 8, b), "misaligned"),
        "tensor-out-of-bounds": (_u("Q", small[0] + 80, (dlen + 63) // 64 * 64, b), "out-of-bounds"),
        "overlapping-tensors": (_u("Q", small[0] + 80, by_off[by_off.index(small) - 1][3], b), "overlap"),
    }
    # hole: the last tensor in data order one row shorter (shape and length
    # kept consistent), so the section no longer ends at the last tensor
    p, dt, dims, off, ln = last
    _, be, bb = container.DTYPES[dt]
    row = (dims[-1] // be * bb) if len(dims) > 1 else (be and bb)
    hb = _u("Q", p + 16, dims[0] - 1, b)
    hb = _u("Q", p + 88, ln - (row if len(dims) > 1 else bb), hb)
    cases["hole-in-weights"] = (hb, "non-canonical-layout")
    return cases


CASES = hostile()


@pytest.mark.parametrize("name", sorted(CASES))
def test_hostile_corpus(tmp_path, name):
    data, code = CASES[name]
    path = tmp_path / (name + ".mim")
    path.write_bytes(data)
    with pytest.raises(container.MimError) as e:
        container.MimFile(str(path)).close()
    assert e.value.code == code, str(e.value)


def test_altered_weights_fail_hash_verification(tmp_path):
    b = bytearray(RAW)
    doff = struct.unpack_from("<Q", b, 32)[0]
    b[doff + 100] ^= 0xFF
    path = tmp_path / "altered.mim"
    path.write_bytes(bytes(b))
    f = container.MimFile(str(path))  # opens
    with pytest.raises(container.MimError) as e:
        f.verify_hashes()
    f.close()
    assert e.value.code == "hash-mismatch"
