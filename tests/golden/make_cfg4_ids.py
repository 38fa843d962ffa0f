"""Writes cfg4_ids.json: the CPU restatement's greedy ids for BASELINE
config 4 at its stated size, for tests/test_gpu_decoder.py.

Config 4's model is the Llama-3-8B shape (32 layers, d 4096, FFN 14336,
32/8 heads, vocab 128256) with random Q4_K_M weights. The weights are drawn
and encoded on the device (synthetic.build, seed 3, the same call the GPU
tests make), so this script needs a GPU: it builds them, downloads their
bytes and runs oracle/llama_ref.py (the C restatement of the reference's
numerics, f16 cache, 8-bit activations in blocks of 256) over a 512-token
prompt of uniform ids (seed 7, the first of eight drawn in a row) and 32
greedy steps (reference cmd/mim-run/main.go:184-257). The prompt runs
through the restatement in chunks of 64 rows: every row's arithmetic is its
own (the cache holds the earlier rows' keys and values), so the ids are
those of one 512-row pass.

The fixture holds the ids, the prompt's seed and length, and SHA-256
digests of three of the matrices, so that a test can tell whether the
device still builds the same weight bytes.

Usage (from the repository root, on a GPU box, about two minutes of CPU):
    python tests/golden/make_cfg4_ids.py [output path]
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for sub in ("mimir-model_amd", "oracle"):
    if os.path.join(ROOT, sub) not in sys.path:
        sys.path.insert(0, os.path.join(ROOT, sub))

WEIGHT_SEED = 3
PROMPT_SEED = 7
PROMPT_LEN = 512
N_NEW = 32
SLOTS = 8
DIGESTED = ("blk.0.attn_q.weight", "blk.31.ffn_down.weight", "output.weight")
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg4_ids.json")


def prompts(vocab):
    """The eight 512-token prompts (uniform ids, drawn in a row from seed 7);
    the first is the batch-1 prompt."""
    rng = np.random.default_rng(PROMPT_SEED)
    return np.stack([rng.integers(0, vocab, PROMPT_LEN) for _ in range(SLOTS)]).astype(np.int32)


def digests(host):
    """SHA-256 of the block bytes of the DIGESTED matrices ({name: (dtype,
    shape, bytes)} as synthetic.host_bytes returns)."""
    return {name: hashlib.sha256(np.ascontiguousarray(host[name][2]).tobytes()).hexdigest() for name in DIGESTED}


def main(out):
    import llama_ref
    import synthetic

    t0 = time.time()
    cfg = dict(synthetic.LLAMA_8B, context=PROMPT_LEN + N_NEW)
    tensors = synthetic.build(cfg, seed=WEIGHT_SEED)
    host = synthetic.host_bytes(tensors)
    for _, _, w in tensors.values():
        if hasattr(w, "release"):
            w.release()
    print(f"weights built and downloaded ({time.time() - t0:.0f} s)", flush=True)
    ref = llama_ref.Decoder(llama_ref.Model(cfg, host), a8=True, cache_f16=True, threads=16)
    prompt = prompts(cfg["vocab"])[0]
    for c0 in range(0, PROMPT_LEN, 64):
        last = c0 + 64 >= PROMPT_LEN
        lg = ref.forward(prompt[c0:c0 + 64], np.arange(c0, c0 + 64), last_only=last)
        print(f"prompt rows {c0}..{c0 + 63} ({time.time() - t0:.0f} s)", flush=True)
    lg = lg[-1]
    ids = []
    for i in range(N_NEW):
        ids.append(llama_ref.argmax(lg))
        if i + 1 < N_NEW:
            lg = ref.forward([ids[-1]], [PROMPT_LEN + i])[0]
        print(f"id {i}: {ids[-1]} ({time.time() - t0:.0f} s)", flush=True)
    fixture = {"model": "synthetic.LLAMA_8B, synthetic.build(seed=3), Q4_K_M", "prompt_seed": PROMPT_SEED,
               "prompt_len": PROMPT_LEN, "n_new": N_NEW, "cache": "f16", "activations": "a8, blocks of 256",
               "ids": ids, "weights_sha256": digests(host)}
    with open(out, "w") as f:
        json.dump(fixture, f, indent=1)
    print(f"wrote {out}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else FIXTURE)
