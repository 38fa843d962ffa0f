"""Writes the golden fixtures of tests/golden/ from the reference's own test
data (run once, in the build container; the GPU box never reads
/root/reference).

Fixtures (data only: inputs and expected outputs):
  quant_golden.json        q8_0, q4_k, q6_k entries of the reference's
                           testdata/quant_golden.json (block bytes, f32 input
                           bits for q8_0, expected f32 bits; produced by the
                           gguf package, reference tools/gen_quant_golden.py).
  dequantize_cases.json    the q8_0/q4_k/q6_k "to_f32" cases of the reference's
                           conformance corpus
                           (testdata/conformance/primitives/dequantize.json).
  llama_tensors.npz        raw block bytes and shapes of the Q4_K and Q6_K
                           tensors of testdata/llama/tiny-q4km.gguf (blocks
                           written by llama.cpp's quantizer), read with a
                           minimal GGUF v3 header parser.
  {llama,qwen2}_model.npz  every tensor of testdata/{llama,qwen2}/tiny-q4km.gguf
                           (block bytes, or f32 values), for the decoder tests.
  {llama,qwen2}_expected.json  the model configuration read from the GGUF
                           metadata and the reference's expected outputs
                           (testdata/*/expected.json: prompt ids, greedy ids,
                           float64-oracle logits, llama.cpp's deviation).
  {llama,qwen2}-tiny-q4km.gguf  the reference's GGUF fixtures
                           (testdata/{llama,qwen2}/tiny-q4km.gguf, written by
                           llama.cpp), copied byte for byte, for the
                           product's own GGUF reader.
  tiny-llama.mim, tiny-llama.expected.json
                           the reference's compatibility fixture
                           (testdata/compat/0.2-0.1/): a container written by
                           its importer and the Go executor's logits for two
                           runs, copied byte for byte.

Usage: python tests/golden/make_golden.py [/root/reference]
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def gguf_tensors(path, with_meta=False):
    """Returns {name: (ggml_type, shape, raw bytes)} of a GGUF v2/v3 file
    (and the metadata dict, with_meta)."""
    with open(path, "rb") as f:
        data = f.read()
    off = 0

    def rd(fmt):
        nonlocal off
        v = struct.unpack_from("<" + fmt, data, off)
        off += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def rstr():
        nonlocal off
        n = rd("Q")
        s = data[off:off + n].decode("utf-8", errors="replace")
        off += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def rval(t):
        if t in scalar:
            return rd(scalar[t])
        if t == 8:
            return rstr()
        if t == 9:
            et, n = rd("I"), rd("Q")
            return [rval(et) for _ in range(n)]
        raise ValueError(f"gguf value type {t}")

    assert data[:4] == b"GGUF", "not a GGUF file"
    off = 4
    version = rd("I")
    assert version in (2, 3), version
    n_tensors, n_kv = rd("Q"), rd("Q")
    align = 32
    meta = {}
    for _ in range(n_kv):
        key = rstr()
        t = rd("I")
        v = rval(t)
        if not key.startswith("tokenizer."):
            meta[key] = v
        if key == "general.alignment":
            align = int(v)
    infos = []
    for _ in range(n_tensors):
        name = rstr()
        nd = rd("I")
        dims = [rd("Q") for _ in range(nd)]
        t = rd("I")
        o = rd("Q")
        infos.append((name, dims, t, o))
    base = (off + align - 1) // align * align
    # block sizes of the ggml types used here
    sizes = {0: (1, 4), 8: (32, 34), 12: (256, 144), 14: (256, 210)}
    out = {}
    for name, dims, t, o in infos:
        if t not in sizes:
            continue
        be, bb = sizes[t]
        n = int(np.prod(dims))
        nbytes = n // be * bb
        out[name] = (t, [int(d) for d in reversed(dims)], data[base + o: base + o + nbytes])
    return (out, meta) if with_meta else out


def write_model(ref, fx):
    """The decoder fixtures of testdata/<fx> (model tensors, config, expected)."""
    t, meta = gguf_tensors(os.path.join(ref, f"testdata/{fx}/tiny-q4km.gguf"), with_meta=True)
    arrays = {}
    for name, (gt, shape, raw) in sorted(t.items()):
        key = name.replace(".", "_")
        if gt == 0:
            arrays[key + "__f32"] = np.frombuffer(raw, np.float32).reshape(shape)
        else:
            arrays[key + "__bytes"] = np.frombuffer(raw, np.uint8)
            arrays[key + "__dtype"] = np.array([{8: 64, 12: 66, 14: 67}[gt]], np.int64)
        arrays[key + "__shape"] = np.array(shape, np.int64)
    np.savez_compressed(os.path.join(HERE, f"{fx}_model.npz"), **arrays)
    arch = meta["general.architecture"]
    cfg = {
        "arch": arch,
        "layers": meta[f"{arch}.block_count"],
        "embed": meta[f"{arch}.embedding_length"],
        "ffn": meta[f"{arch}.feed_forward_length"],
        "heads": meta[f"{arch}.attention.head_count"],
        "kv_heads": meta.get(f"{arch}.attention.head_count_kv", meta[f"{arch}.attention.head_count"]),
        "rope_dims": meta.get(f"{arch}.rope.dimension_count"),
        "rope_theta": meta.get(f"{arch}.rope.freq_base", 10000.0),
        "norm_eps": meta[f"{arch}.attention.layer_norm_rms_epsilon"],
        "context": meta[f"{arch}.context_length"],
    }
    e = json.load(open(os.path.join(ref, f"testdata/{fx}/expected.json")))
    out = {"config": cfg, "vocab": e["vocab"], "prompt_ids": e["prompt_ids"], "greedy": e["greedy"],
           "prompt_logits": e["prompt_logits"], "greedy_logits": e["greedy_logits"],
           "llama_cpp_max_diff": e["llama_cpp_max_diff"]}
    json.dump(out, open(os.path.join(HERE, f"{fx}_expected.json"), "w"))
    print("wrote", fx, cfg)


def main(ref):
    g = json.load(open(os.path.join(ref, "testdata/quant_golden.json")))
    json.dump({k: g[k] for k in ("q8_0", "q4_k", "q6_k")}, open(os.path.join(HERE, "quant_golden.json"), "w"))

    c = json.load(open(os.path.join(ref, "testdata/conformance/primitives/dequantize.json")))
    keep = [case for case in c["cases"] if case["name"] in ("q8_0/to_f32", "q4_k/to_f32", "q6_k/to_f32")]
    json.dump({"op": c["op"], "cases": keep}, open(os.path.join(HERE, "dequantize_cases.json"), "w"), indent=1)

    t = gguf_tensors(os.path.join(ref, "testdata/llama/tiny-q4km.gguf"))
    arrays = {}
    names = []
    for name, (gt, shape, raw) in sorted(t.items()):
        if gt not in (12, 14):
            continue
        key = name.replace(".", "_")
        names.append(name)
        arrays[key + "__bytes"] = np.frombuffer(raw, np.uint8)
        arrays[key + "__shape"] = np.array(shape, np.int64)
        arrays[key + "__dtype"] = np.array([66 if gt == 12 else 67], np.int64)
    np.savez_compressed(os.path.join(HERE, "llama_tensors.npz"), **arrays)
    print("wrote", len(names), "tensors:", ", ".join(names))
    for fx in ("llama", "qwen2"):
        write_model(ref, fx)
    for fx in ("llama", "qwen2"):
        with open(os.path.join(ref, f"testdata/{fx}/tiny-q4km.gguf"), "rb") as f:
            data = f.read()
        with open(os.path.join(HERE, f"{fx}-tiny-q4km.gguf"), "wb") as f:
            f.write(data)
        print("copied", fx, "gguf", len(data), "bytes")
    for name in ("tiny-llama.mim", "tiny-llama.expected.json"):
        with open(os.path.join(ref, "testdata/compat/0.2-0.1", name), "rb") as f:
            data = f.read()
        with open(os.path.join(HERE, name), "wb") as f:
            f.write(data)
        print("copied", name, len(data), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
