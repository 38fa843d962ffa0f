"""Random llama-shaped models built on the device, for the decode
benchmarks: a Llama-3.2-1B shape (16 layers, d 2048, FFN 8192, 32/8 heads,
vocab 128256, theta 500000) and a Llama-3-8B shape (32 layers, d 4096,
FFN 14336, 32/8 heads, vocab 128256). Weights are N(0, 0.02^2) drawn on the
GPU and encoded as Q4_K_M: Q4_K for the embedding, q, k, o, gate and up,
Q6_K for v, down and the output head. Norm scales are ones.

The matrices are drawn, encoded and registered one at a time, so building
needs device memory for the weights plus one f32 copy of the largest
matrix; nothing passes through host memory.
"""
import numpy as np

import hiprt
import mimg

LLAMA_1B = dict(arch="llama", layers=16, embed=2048, ffn=8192, heads=32, kv_heads=8, rope_theta=500000.0,
                norm_eps=1e-5, vocab=128256)
LLAMA_8B = dict(arch="llama", layers=32, embed=4096, ffn=14336, heads=32, kv_heads=8, rope_theta=500000.0,
                norm_eps=1e-5, vocab=128256)


def matrices(cfg):
    """[(GGUF name, dtype, N, K)] of a llama model's weight matrices."""
    E, F, H, Hkv, V = cfg["embed"], cfg["ffn"], cfg["heads"], cfg["kv_heads"], cfg["vocab"]
    D = E // H
    out = [("token_embd.weight", mimg.Q4_K, V, E)]
    for l in range(cfg["layers"]):
        p = f"blk.{l}."
        out += [(p + "attn_q.weight", mimg.Q4_K, H * D, E), (p + "attn_k.weight", mimg.Q4_K, Hkv * D, E),
                (p + "attn_v.weight", mimg.Q6_K, Hkv * D, E), (p + "attn_output.weight", mimg.Q4_K, E, H * D),
                (p + "ffn_gate.weight", mimg.Q4_K, F, E), (p + "ffn_up.weight", mimg.Q4_K, F, E),
                (p + "ffn_down.weight", mimg.Q6_K, E, F)]
    out.append(("output.weight", mimg.Q6_K, V, E))
    return out


def weight_bytes(cfg, per_token=False):
    """Bytes of the matrices (per_token: those a decode step reads, i.e. all
    but the embedding table, of which it reads one row)."""
    total = 0
    for name, dt, n, k in matrices(cfg):
        rb = mimg.row_bytes(dt, k)
        total += rb if (per_token and name == "token_embd.weight") else n * rb
    return total


def build(cfg, seed=0, std=0.02, log=None):
    """{name: (dtype, shape, data)} for decoder.Decoder: registered device
    weights and f32 norm scales."""
    mimg.init()
    stream = hiprt.Stream()
    mats = matrices(cfg)
    big = max(n * k for _, _, n, k in mats)
    f32 = hiprt.DeviceBuffer(big * 4)
    enc = hiprt.DeviceBuffer(max(n * mimg.row_bytes(dt, k) for _, dt, n, k in mats))
    tensors = {}
    for i, (name, dt, n, k) in enumerate(mats):
        nbytes = n * mimg.row_bytes(dt, k)
        mimg.synthetic_normal_dev(seed * 1000003 + i, std, f32.ptr, n * k, stream.handle)
        mimg.quantize_dev(dt, f32.ptr, n * k, enc.ptr, nbytes, stream.handle)
        stream.sync()
        tensors[name] = (dt, [n, k], mimg.Weight((enc.ptr, nbytes), dt, n, k, device=True))
    f32.free()
    enc.free()
    ones = np.ones(cfg["embed"], np.float32)
    for l in range(cfg["layers"]):
        tensors[f"blk.{l}.attn_norm.weight"] = (mimg.F32, [cfg["embed"]], ones)
        tensors[f"blk.{l}.ffn_norm.weight"] = (mimg.F32, [cfg["embed"]], ones)
    tensors["output_norm.weight"] = (mimg.F32, [cfg["embed"]], ones)
    if log:
        log(f"  built {cfg['layers']}-layer model: {weight_bytes(cfg) / 1e9:.2f} GB of weights")
    return tensors


def host_bytes(tensors):
    """The block bytes of every matrix, downloaded (for the CPU restatement)."""
    out = {}
    for name, (dt, shape, w) in tensors.items():
        if isinstance(w, mimg.Weight):
            ptr, _ = w.info()
            nbytes = shape[0] * mimg.row_bytes(dt, shape[1])
            arr = np.empty(nbytes, np.uint8)
            hiprt.check(hiprt.rt().hipMemcpy(arr.ctypes.data, ptr, nbytes, hiprt.D2H), "D2H")
            out[name] = (dt, shape, arr)
        else:
            out[name] = (dt, shape, w)
    return out
