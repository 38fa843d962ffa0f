"""CPU restatement of the reference's llama/qwen2 forward pass: the graph
BuildLlama writes (reference importer/llama.go:317-547) run with the interp
fast paths. TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's
baseline, never by the product (libmimg and the GPU decoder).

Each op follows the reference's fast path:
  embedding.v1   a row of token_embd decoded (interp/fast.go:818-842, mim.Dequantize)
  rms_norm.v1    f64 sum of squares, inv = f32(1/sqrt(f64(f32(ss/n)) + f64(f32(eps)))),
                 y = (x*inv)*scale in f32 (interp/fast.go:434-485)
  rope.v1        invFreq_i = theta^(-2i/r) (f64), c, s = f32(cos/sin(pos*invFreq_i)),
                 x1*c - x2*s, x2*c + x1*s in f32; adjacent pairs for llama
                 ("interleaved"), halves for qwen2 (interp/fast.go:507-557,
                 transformer.go:257-324)
  attention.v1/2 keys j <= position visible (the graph's mask); attendRow
                 with the AVX2 kernels: scores, Cephes expf sum, ordered
                 weighted sum (interp/fast.go:559-751, attn_amd64.s), the C
                 restatement mimref.attention; GQA head h reads kv head
                 h/(H/Hkv); with the cache in f16 the new keys and values are
                 rounded to f16 as they are stored (llama.go:489-499)
  swiglu.v1      SiluMulF32 over the pieces of parallel() for GOMAXPROCS =
                 procs (interp/fast.go:487-498, attn.go:63-76), mimref.silu_mul
  linears        dequant_matmul_a8.v2 (block 256) for Q4_K/Q6_K, v1 (block
                 32) otherwise, with a8; dequant_matmul.v1 without
                 (llama.go:264-280); the oracle's C linear_a8/linear_f32.
The f64 sums of rms_norm use numpy's order and the f64 cos/sin/exp come
from numpy/libm rather than Go's math package: after rounding to f32 these
agree with the reference except with probability ~1e-7 per value. Checks:
the reference fixtures' tolerances (float64-oracle logits) and
tests/test_oracle_decoder.py.
"""
import numpy as np

import mimref

F32, Q8_0, Q4_K, Q6_K = 1, 64, 66, 67


class Model:
    """Config dict and tensors {name: (dtype, shape, bytes | f32 array)}."""

    def __init__(self, config, tensors):
        self.c = dict(config)
        self.t = tensors
        c = self.c
        c.setdefault("kv_heads", c["heads"])
        c["head_dim"] = c["embed"] // c["heads"]
        if not c.get("rope_dims"):
            c["rope_dims"] = c["head_dim"]
        emb = tensors["token_embd.weight"]
        c["vocab"] = emb[1][0]


def rms_norm(x, scale, eps):
    x = np.asarray(x, np.float32)
    n = x.shape[-1]
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1)
    inv = (1.0 / np.sqrt(np.float32(ss / n).astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    y = (x * inv[:, None]).astype(np.float32)
    return (y * scale).astype(np.float32)


def rope_tables(positions, rotary, theta):
    h = rotary // 2
    inv = np.array([theta ** (-2.0 * i / rotary) for i in range(h)], np.float64)
    ang = np.asarray(positions, np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x, cos, sin, rotary, interleaved):
    """x: [T, heads, D] f32; cos/sin: [T, rotary/2]."""
    y = x.copy()
    h = rotary // 2
    if interleaved:
        i1, i2 = np.arange(h) * 2, np.arange(h) * 2 + 1
    else:
        i1, i2 = np.arange(h), np.arange(h) + h
    x1, x2 = x[:, :, i1], x[:, :, i2]
    c, s = cos[:, None, :], sin[:, None, :]
    y[:, :, i1] = (x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)
    y[:, :, i2] = (x2 * c).astype(np.float32) + (x1 * s).astype(np.float32)
    return y


def attention(q, kc, vc, positions, kv_heads, kstart=None):
    """q: [T, H, D]; kc/vc: [Hkv, C, D] float32 or float16; query t sees
    cache entries kstart[t] (default 0) .. positions[t]."""
    return mimref.attention(q, kc, vc, np.asarray(positions, np.int64), kstart)


def swiglu(g, u, procs=16):
    return mimref.silu_mul(g, u, procs).reshape(np.shape(g))


class Decoder:
    """The forward pass with a key-value cache, on the CPU."""

    def __init__(self, model, a8=True, cache_f16=False, threads=8, procs=16, kquant_block=256):
        self.m, self.a8, self.f16, self.threads, self.procs = model, a8, cache_f16, threads, procs
        self.kquant_block = kquant_block
        c = model.c
        C = c["context"]
        cdt = np.float16 if cache_f16 else np.float32
        self.kc = [np.zeros((c["kv_heads"], C, c["head_dim"]), cdt) for _ in range(c["layers"])]
        self.vc = [np.zeros((c["kv_heads"], C, c["head_dim"]), cdt) for _ in range(c["layers"])]

    def linear(self, x, name, bias=None):
        dt, shape, w = self.m.t[name]
        n, k = shape
        if dt == F32:
            y = (x @ w.T).astype(np.float32)
            return y if bias is None else (y + bias).astype(np.float32)
        if self.a8:
            block = self.kquant_block if dt in (Q4_K, Q6_K) else 32
            return mimref.linear_a8(x, w, dt, n, k, bias=bias, block=block, threads=self.threads)
        return mimref.linear_f32(x, w, dt, n, k, bias=bias, threads=self.threads)

    def embed(self, tokens):
        dt, shape, w = self.m.t["token_embd.weight"]
        V, E = shape
        if dt == F32:
            return w[np.asarray(tokens)].astype(np.float32)
        rb = len(w) // V
        return np.stack([mimref.dequantize(dt, w[rb * t: rb * (t + 1)], E) for t in tokens]).astype(np.float32)

    def forward(self, tokens, positions, last_only=False):
        """Logits [T, vocab] for tokens at positions (the cache is updated);
        last_only: the last row's logits only, [1, vocab] (each row of the
        head's product is computed alone, so it is that row of the full
        result)."""
        m, c = self.m, self.m.c
        T, H, Hkv, D = len(tokens), c["heads"], c["kv_heads"], c["head_dim"]
        positions = np.asarray(positions, np.int64)
        cos, sin = rope_tables(positions, c["rope_dims"], c["rope_theta"])
        inter = c["arch"] != "qwen2"
        x = self.embed(tokens)
        for l in range(c["layers"]):
            p = f"blk.{l}."
            bias = (lambda nm: m.t[p + nm][2] if (p + nm) in m.t else None)
            h = rms_norm(x, m.t[p + "attn_norm.weight"][2], c["norm_eps"])
            q = self.linear(h, p + "attn_q.weight", bias("attn_q.bias")).reshape(T, H, D)
            k = self.linear(h, p + "attn_k.weight", bias("attn_k.bias")).reshape(T, Hkv, D)
            v = self.linear(h, p + "attn_v.weight", bias("attn_v.bias")).reshape(T, Hkv, D)
            q = rope(q, cos, sin, c["rope_dims"], inter)
            k = rope(k, cos, sin, c["rope_dims"], inter)
            for i, pos in enumerate(positions):
                self.kc[l][:, pos] = k[i]  # rounded to f16 (RNE) with an f16 cache
                self.vc[l][:, pos] = v[i]
            o = attention(q, self.kc[l], self.vc[l], positions, Hkv).reshape(T, H * D)
            x = (x + self.linear(o, p + "attn_output.weight")).astype(np.float32)
            h = rms_norm(x, m.t[p + "ffn_norm.weight"][2], c["norm_eps"])
            a = swiglu(self.linear(h, p + "ffn_gate.weight"), self.linear(h, p + "ffn_up.weight"), self.procs)
            x = (x + self.linear(a, p + "ffn_down.weight")).astype(np.float32)
        if last_only:
            x = x[-1:]
        x = rms_norm(x, m.t["output_norm.weight"][2], c["norm_eps"])
        head = "output.weight" if "output.weight" in m.t else "token_embd.weight"
        return self.linear(x, head)


def argmax(v):
    """First index of the largest value (reference cmd/mim-run/main.go:184-192)."""
    return int(np.argmax(v))
