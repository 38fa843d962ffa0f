"""The reference's tiny llama/qwen2 fixtures (tests/golden/*_model.npz and
*_expected.json, written by tests/golden/make_golden.py from the reference's
testdata/{llama,qwen2}) and the checks of its generate tests
(reference cmd/mim-run/main_test.go:125-140, 178-257)."""
import base64
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32 = 1
FIXTURES = ("llama", "qwen2")


def _key_to_name(key):
    # blk_0_attn_q_weight -> blk.0.attn_q.weight (the GGUF tensor names)
    parts = key.split("_")
    for suf in ("_weight", "_bias"):
        if key.endswith(suf):
            stem = key[:-len(suf)]
            if parts[0] == "blk":
                stem = f"blk.{parts[1]}." + "_".join(stem.split("_")[2:])
            return f"{stem}.{suf[1:]}"
    return key


def load(name):
    """(config dict, {tensor name: (dtype, shape, data)}, expected dict)."""
    e = json.load(open(os.path.join(GOLDEN, f"{name}_expected.json")))
    z = np.load(os.path.join(GOLDEN, f"{name}_model.npz"))
    tensors = {}
    for key in sorted({k.rsplit("__", 1)[0] for k in z.files}):
        shape = [int(v) for v in z[key + "__shape"]]
        if key + "__f32" in z.files:
            tensors[_key_to_name(key)] = (F32, shape, np.ascontiguousarray(z[key + "__f32"], np.float32))
        else:
            tensors[_key_to_name(key)] = (int(z[key + "__dtype"][0]), shape, np.ascontiguousarray(z[key + "__bytes"]))
    return dict(e["config"]), tensors, e


def f32b64(s):
    """Logits stored as base64 little-endian f32 (reference main_test.go f32b64)."""
    return np.frombuffer(base64.b64decode(s), np.float32)


def near(got, want, tol):
    """max |got - want| <= tol * max |want| (reference main_test.go:125-140).
    Returns (ok, worst, allowed)."""
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    assert got.size == want.size, (got.size, want.size)
    worst = float(np.max(np.abs(got - want)))
    allowed = tol * float(np.max(np.abs(want)))
    return worst <= allowed and not np.isnan(worst), worst, allowed


def max_diff(got, want):
    return float(np.max(np.abs(np.asarray(got, np.float64).ravel() - np.asarray(want, np.float64).ravel())))
