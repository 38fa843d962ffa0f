"""The product's GGUF reader (mimir-model_amd/gguf.py) on the reference's
GGUF fixtures: every llama tensor's bytes hash to the SHA-256 the
reference's compatibility fixture lists for the container its importer
wrote from this file (testdata/compat/0.2-0.1/tiny-llama.expected.json),
with the same dtype and shape; the decoder configuration equals the one
the importer wrote; the bytes equal the decoder fixtures'; malformed files
are rejected as ParseGGUF rejects them (importer/gguf.go:304-460)."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import container
import decoder
import fixture_models as fm
import gguf
from conftest import GOLDEN

EXPECTED = json.load(open(os.path.join(GOLDEN, "tiny-llama.expected.json")))


def path(fx):
    return os.path.join(GOLDEN, f"{fx}-tiny-q4km.gguf")


def test_llama_tensors_equal_the_imported_container():
    g = gguf.GGUFFile(path("llama"))
    want = {t["name"]: t for t in EXPECTED["tensors"] if not t["name"].startswith("mim.")}
    assert sorted(t.name for t in g.tensors) == sorted(want)
    for t in g.tensors:
        w = want[t.name]
        assert container.DTYPES[t.dtype][0] == w["dtype"] and t.shape == w["shape"], t.name
        assert hashlib.sha256(g.tensor_bytes(t.name)).hexdigest() == w["sha256"], t.name
    g.close()


@pytest.mark.parametrize("fx", fm.FIXTURES)
def test_config_and_bytes_match_the_fixtures(fx):
    g = gguf.GGUFFile(path(fx))
    cfg = decoder.config_from_metadata(g.metadata)
    want, tensors, _ = fm.load(fx)
    for k in ("arch", "layers", "embed", "ffn", "heads", "kv_heads", "rope_dims", "context"):
        assert cfg[k] == want[k], k
    assert cfg["rope_theta"] == pytest.approx(want["rope_theta"]) and cfg["norm_eps"] == pytest.approx(want["norm_eps"])
    for name, (dt, shape, data) in tensors.items():
        t = g.by_name[name]
        assert t.dtype == dt and t.shape == shape, name
        got = np.frombuffer(g.tensor_bytes(name), np.uint8)
        assert np.array_equal(got, np.asarray(data).view(np.uint8).ravel()), name
    g.close()


RAW = open(path("llama"), "rb").read()


def _tensor_table_offset(b):
    """Offset of the first tensor info (after the metadata)."""
    r = gguf._Reader(memoryview(b))
    r.take(4)
    r.u("I", 4)
    nt, nkv = r.u("Q", 8), r.u("Q", 8)
    for _ in range(nkv):
        r.str()
        t = r.u("I", 4)
        r.value(t, 0)
    return r.off


def _first_tensor_type_offset(b):
    off = _tensor_table_offset(b)
    n = struct.unpack_from("<Q", b, off)[0]
    nd = struct.unpack_from("<I", b, off + 8 + n)[0]
    return off + 8 + n + 4 + 8 * nd  # the ggml type u32


@pytest.mark.parametrize("name,data,msg", [
    ("bad-magic", b"GGUX" + RAW[4:], "bad magic"),
    ("big-endian", RAW[:4] + struct.pack(">I", 3) + RAW[8:], "big-endian"),
    ("version", RAW[:4] + struct.pack("<I", 7) + RAW[8:], "unsupported version"),
    ("truncated", RAW[:_tensor_table_offset(RAW) + 10], "truncated"),
    ("too-many-tensors", RAW[:8] + struct.pack("<Q", 1 << 30) + RAW[16:], "do not fit"),
])
def test_malformed_headers(tmp_path, name, data, msg):
    p = tmp_path / name
    p.write_bytes(data)
    with pytest.raises(gguf.GGUFError) as e:
        gguf.GGUFFile(str(p)).close()
    assert msg in str(e.value)


def test_unknown_and_unsupported_types(tmp_path):
    off = _first_tensor_type_offset(RAW)
    for gt, msg in ((13, "type Q5_K, which mim does not define"), (77, "unknown type 77")):
        b = bytearray(RAW)
        struct.pack_into("<I", b, off, gt)
        p = tmp_path / f"t{gt}.gguf"
        p.write_bytes(bytes(b))
        with pytest.raises(gguf.GGUFError) as e:
            gguf.GGUFFile(str(p)).close()
        assert msg in str(e.value)


def test_tensor_outside_the_file(tmp_path):
    off = _first_tensor_type_offset(RAW) + 4  # the tensor's data offset
    b = bytearray(RAW)
    struct.pack_into("<Q", b, off, (len(RAW) + 31) // 32 * 32)
    p = tmp_path / "oob.gguf"
    p.write_bytes(bytes(b))
    with pytest.raises(gguf.GGUFError) as e:
        gguf.GGUFFile(str(p)).close()
    assert "outside the file" in str(e.value)


def test_config_rejections():
    g = gguf.GGUFFile(path("llama"))
    md = dict(g.metadata)
    g.close()
    bad = dict(md, **{"general.architecture": "gpt2"})
    with pytest.raises(ValueError, match="only"):
        decoder.config_from_metadata(bad)
    bad = dict(md, **{"llama.attention.head_count_kv": 3})
    with pytest.raises(ValueError, match="do not divide"):
        decoder.config_from_metadata(bad)
    bad = dict(md, **{"llama.rope.scaling.type": "yarn"})
    with pytest.raises(ValueError, match="not supported"):
        decoder.config_from_metadata(bad)
    assert decoder.config_from_metadata(md, context=32)["context"] == 32
