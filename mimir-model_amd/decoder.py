"""Greedy llama/qwen2 decoding with every op on the GPU, through libmimg.

The forward pass is the graph the reference's importer writes for a llama
or qwen2 model (reference importer/llama.go:317-547) run the way its interp
fast paths run it: embedding.v1, rms_norm.v1, the quantized linears
(dequant_matmul_a8.v2 / .v1 with 8-bit activations, dequant_matmul.v1
without), rope.v1, the cache scatter, attention.v1/.v2 with the causal and
slot mask, swiglu.v1, and the greedy loop of cmd/mim-run/main.go:184-257.
Activations, the key-value cache and the chosen tokens stay in device
memory; a decode step is one HIP graph replay with no host round trip.

Several sequences ("slots", reference LlamaOptions.Slots,
importer/llama.go:306-310) share one cache of slots * context positions:
the token at position p of slot s goes to cache index s*context + p and sees
the keys s*context .. s*context + p.

There is no CPU fallback: every op is a libmimg call, which raises if the
library or a gfx950 GPU is missing.
"""
import numpy as np

import hiprt
import mimg

F32 = mimg.F32


class Config:
    """The model shape (reference importer/llama.go LlamaConfig)."""

    def __init__(self, arch="llama", layers=1, embed=256, ffn=256, heads=4, kv_heads=None, rope_dims=None,
                 rope_theta=10000.0, norm_eps=1e-5, context=64, **_):
        self.arch, self.layers, self.embed, self.ffn = arch, int(layers), int(embed), int(ffn)
        self.heads = int(heads)
        self.kv_heads = int(kv_heads or heads)
        self.head_dim = self.embed // self.heads
        self.rope_dims = int(rope_dims or self.head_dim)
        self.rope_theta, self.norm_eps, self.context = float(rope_theta), float(norm_eps), int(context)
        # llama rotates adjacent pairs, qwen2 the two halves
        # (reference interp/transformer.go:257-324)
        self.interleaved = arch != "qwen2"
        if self.embed % self.heads or self.heads % self.kv_heads or self.rope_dims % 2:
            raise ValueError(f"inconsistent shape: embed {embed}, heads {heads}, kv heads {kv_heads}, rope {rope_dims}")


MAX_CONTEXT = 1 << 20


def config_from_metadata(md, context=0):
    """The decoder shape of a llama or qwen2 model from its metadata, as the
    reference's importer reads it (importer/llama.go LlamaConfigOf): the
    required keys must be positive and at most 2^24, head counts must
    divide, rope scaling is not supported, the context is the model's own
    unless given."""
    arch = md.get("general.architecture")
    if arch not in ("llama", "qwen2"):
        raise ValueError(f'architecture {arch!r}: only "llama" and "qwen2" graphs can be built')

    def req(key):
        v = md.get(f"{arch}.{key}")
        if isinstance(v, bool) or not isinstance(v, int) or v <= 0 or v > 1 << 24:
            raise ValueError(f"metadata {arch}.{key} is missing or invalid")
        return v

    c = dict(arch=arch, layers=req("block_count"), embed=req("embedding_length"), ffn=req("feed_forward_length"),
             heads=req("attention.head_count"))
    max_ctx = req("context_length")
    c["kv_heads"] = req("attention.head_count_kv") if f"{arch}.attention.head_count_kv" in md else c["heads"]
    if c["embed"] % c["heads"] or c["heads"] % c["kv_heads"]:
        raise ValueError(f"embedding length {c['embed']}, {c['heads']} heads and {c['kv_heads']} key-value heads "
                         "do not divide")
    head_dim = c["embed"] // c["heads"]
    c["rope_dims"] = head_dim
    if f"{arch}.rope.dimension_count" in md:
        c["rope_dims"] = req("rope.dimension_count")
        if c["rope_dims"] % 2 or c["rope_dims"] > head_dim:
            raise ValueError(f"rope dimension count {c['rope_dims']} for head size {head_dim}")
    c["rope_theta"] = float(md.get(f"{arch}.rope.freq_base", 10000.0))
    t = md.get(f"{arch}.rope.scaling.type")
    if isinstance(t, str) and t != "none":
        raise ValueError(f"rope scaling {t!r} is not supported yet")
    eps = md.get(f"{arch}.attention.layer_norm_rms_epsilon")
    if not isinstance(eps, float) or eps <= 0:
        raise ValueError(f"metadata {arch}.attention.layer_norm_rms_epsilon is missing or invalid")
    # the importer stores f32 metadata widened to f64; the graph's rms_norm
    # attribute keeps it, and rms_norm.v1 rounds it to f32
    c["norm_eps"] = eps
    c["context"] = context if context > 0 else max_ctx
    if c["context"] > MAX_CONTEXT:
        raise ValueError(f"context length {c['context']} exceeds {MAX_CONTEXT}")
    return c


def inv_freq(cfg):
    """theta^(-2i/r) in f64, i < r/2 (reference interp/fast.go:507-557)."""
    r = cfg.rope_dims
    return np.array([cfg.rope_theta ** (-2.0 * i / r) for i in range(r // 2)], np.float64)


class Decoder:
    """One model on the GPU with its key-value cache.

    tensors: {GGUF tensor name: (dtype, shape, data)}, where data is the
    block bytes (np.uint8) of a quantized matrix, an np.float32 array for a
    norm scale or bias, or an already registered mimg.Weight. procs is the
    GOMAXPROCS of the reference run to reproduce (its swiglu results depend
    on it). kquant_block is the activation block of the Q4_K/Q6_K products
    with 8-bit activations (256: dequant_matmul_a8.v2, 32: .v1).
    f32_tile_rows (float32 activations only): products of at least this many
    rows run on the fp32 matrix cores (mimg_linear_f32_mfma_dev), within the
    spec's bound for dequant_matmul.v1 but not in the reference's float
    order; 0 keeps the reference's order everywhere.
    """

    def __init__(self, config, tensors, a8=True, cache_f16=False, max_rows=64, slots=1, procs=16, kquant_block=256,
                 f32_tile_rows=0, fuse_rope=True, fuse_swiglu=True):
        c = self.c = config if isinstance(config, Config) else Config(**config)
        self.a8, self.f16, self.slots = bool(a8), bool(cache_f16), int(slots)
        # activation blocks for Q4_K/Q6_K weights: 256 is dequant_matmul_a8.v2
        # as the importer writes it (importer/llama.go:264-280), 32 is .v1
        if kquant_block not in (32, 256):
            raise ValueError(f"kquant_block {kquant_block}: 32 or 256")
        self.kquant_block = kquant_block
        self.f32_tile_rows = int(f32_tile_rows)
        # the reference's GOMAXPROCS: swiglu's results follow its piece split
        self.procs = int(procs)
        self.R = int(max_rows)
        mimg.init()
        self.stream = hiprt.Stream()
        self.w, self.vec = {}, {}
        for name, (dt, shape, data) in tensors.items():
            if isinstance(data, mimg.Weight):
                self.w[name] = data
            elif dt == F32:
                if len(shape) != 1:
                    raise mimg.NotHandled(1, f"{name}: f32 matrices are not handled")
                self.vec[name] = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(data, np.float32))
            else:
                self.w[name] = mimg.Weight(data, dt, int(shape[0]), int(shape[1]))
        if c.context > 8192:
            raise ValueError(f"context {c.context}: attention handles at most 8192 positions per sequence")
        self.head = self.w.get("output.weight") or self.w["token_embd.weight"]
        self.vocab = self.w["token_embd.weight"].n
        E, F, H, Hkv, D, R = c.embed, c.ffn, c.heads, c.kv_heads, c.head_dim, self.R
        self.cache_len = self.slots * c.context
        esz = 2 if self.f16 else 4
        B = hiprt.DeviceBuffer
        self.kc = [B(Hkv * self.cache_len * D * esz) for _ in range(c.layers)]
        # the value cache is blocked by eight keys (include/mimg.h)
        self.vc = [B(Hkv * mimg.vcache_len(self.cache_len) * D * esz) for _ in range(c.layers)]
        for buf in self.kc + self.vc:
            buf.zero()
        self.invf = B.from_array(inv_freq(c))
        self.x, self.h, self.ao = B(R * E * 4), B(R * E * 4), B(R * E * 4)
        # the fused norm + q/k/v GEMV writes x + resid to the other buffer
        self.x_pair = (self.x, B(E * 4))
        self.x_alt = self.x_pair[1]
        self.norm_fused = {}  # names -> whether the fused norm GEMV takes them
        # one row: norm, q/k/v, rope and the cache scatter in one launch
        # (until the library answers NotHandled for the shape)
        self.rope_fused = bool(fuse_rope)
        # one row, and 2..8 rows: gate/up products with swiglu in their epilogue
        self.swiglu_fused = bool(fuse_swiglu)
        self.swiglu_rows_fused = bool(fuse_swiglu)
        # 4..8 rows: q/k/v products with rope and the cache scatter
        self.qkv_rows_fused = bool(fuse_rope)
        self.q, self.o = B(R * H * D * 4), B(R * H * D * 4)
        self.k, self.v = B(R * Hkv * D * 4), B(R * Hkv * D * 4)
        self.g, self.u, self.sw = B(R * F * 4), B(R * F * 4), B(R * F * 4)
        self.logits = B(R * self.vocab * 4)
        self.ids, self.pos = B(R * 4), B(R * 8)
        self.cidx, self.kstart = B(R * 8), B(R * 8)
        self.chosen, self.count = B(R * 4), B(4)
        self.out, self.out_cap = None, 0
        kmax = max(E, H * D, F)
        self.ws_bytes = mimg.a8_workspace_bytes(R, kmax)
        self.ws = B(self.ws_bytes)
        self.att_ws_bytes = mimg.attention_workspace_bytes(R, H, c.context)
        self.att_ws = B(self.att_ws_bytes)
        self.graphs = {}

    # ---- the graph's ops ---------------------------------------------------

    def _block(self, w):
        return self.kquant_block if w.dt in (mimg.Q4_K, mimg.Q6_K) else 32

    def _linears(self, names, x, rows, ys, biases=None):
        """ys[i] = x . W_i^T (+ bias_i) for weights sharing the input x."""
        ws = [self.w[n] for n in names]
        bs = [None if b is None or b not in self.vec else self.vec[b].ptr for b in (biases or [None] * len(names))]
        s = self.stream.handle
        if not self.a8:
            tiles = 0 < self.f32_tile_rows <= rows
            for w, b, y in zip(ws, bs, ys):
                (mimg.linear_f32_mfma_dev if tiles else mimg.linear_f32_dev)(w, x, rows, b, y, s)
            return
        blocks = {self._block(w) for w in ws}
        if len(ws) > 1 and len(blocks) == 1:
            mimg.linear_a8_group_dev(ws, x, rows, bs if any(bs) else None, blocks.pop(), ys, self.ws.ptr,
                                     self.ws_bytes, s)
            return
        for w, b, y in zip(ws, bs, ys):
            mimg.linear_a8_dev(w, x, rows, b, self._block(w), y, self.ws.ptr, self.ws_bytes, s)

    def _norm_linears(self, resid, norm, T, names, ys, biases=None, single_fused=False):
        """x += resid; h = rms_norm(x) * scale; ys[i] = h . W_i^T (+ bias_i).
        With 8-bit activations and one block size for the group, the norm
        and the quantization of h are one launch and the products take the
        quantized h (bit for bit the separate ops); at one row, q/k/v
        (single_fused) take one launch for the norm and the products (x +
        resid lands in the other x buffer), or where that kernel does not
        take the shape, the GEMV that quantizes inside."""
        c, s = self.c, self.stream.handle
        E = c.embed
        ws = [self.w[n] for n in names]
        blocks = {self._block(w) for w in ws}
        key = tuple(names)
        if self.a8 and single_fused and T == 1 and blocks == {256} and self.norm_fused.get(key, True):
            # one launch: x + resid into the other x buffer, the norm and the
            # q/k/v products (NotHandled: launched nothing, shape not taken)
            bs = [None if b is None or b not in self.vec else self.vec[b].ptr for b in (biases or [None] * len(names))]
            try:
                mimg.rms_norm_linear_a8_group_dev(ws, self.x.ptr, resid, self.vec[norm].ptr, c.norm_eps,
                                                  self.x_alt.ptr, bs if any(bs) else None, ys, s)
                self.norm_fused[key] = True
                self.x, self.x_alt = self.x_alt, self.x
                return
            except mimg.NotHandled:
                self.norm_fused[key] = False
        if self.a8 and len(blocks) == 1 and not (single_fused and T == 1) and E <= 32768:
            block = blocks.pop()
            mimg.rms_norm_quant_dev(self.x.ptr, resid, self.vec[norm].ptr, c.norm_eps, T, E, self.h.ptr, block,
                                    self.ws.ptr, self.ws_bytes, s)
            bs = [None if b is None or b not in self.vec else self.vec[b].ptr for b in (biases or [None] * len(names))]
            mimg.matmul_a8_quantized_group_dev(ws, self.h.ptr, T, bs if any(bs) else None, block, ys, self.ws.ptr,
                                               self.ws_bytes, s)
            return
        mimg.rms_norm_dev(self.x.ptr, resid, self.vec[norm].ptr, c.norm_eps, T, E, self.h.ptr, s)
        self._linears(names, self.h.ptr, T, ys, biases)

    def _qkv_rope_rows(self, l, resid, qkv, qkv_b, T, pos, cidx):
        """4..8 rows with 8-bit activations of blocks of 256: x += resid and
        the quantized rms_norm (one launch), then the q, k, v products with
        rope and the cache scatter in their epilogues (one launch). False
        (nothing launched) where the library has no such launch."""
        c, s = self.c, self.stream.handle
        p = f"blk.{l}."
        ws = [self.w[n] for n in qkv]
        if not (self.a8 and self.qkv_rows_fused and all(self._block(w) == 256 for w in ws) and c.embed <= 32768
                and c.head_dim in (64, 128) and ws[0].dt == ws[1].dt):
            return False
        bs = [None if b is None or b not in self.vec else self.vec[b].ptr for b in qkv_b]
        mimg.rms_norm_quant_dev(self.x.ptr, resid, self.vec[p + "attn_norm.weight"].ptr, c.norm_eps, T, c.embed,
                                self.h.ptr, 256, self.ws.ptr, self.ws_bytes, s)
        try:
            mimg.matmul_a8_quantized_qkv_rope_kv_dev(ws, self.h.ptr, T, bs if any(bs) else None, 256, self.q.ptr, pos,
                                                     cidx, self.invf.ptr, c.heads, c.kv_heads, c.head_dim,
                                                     c.rope_dims, c.interleaved, self.cache_len, self.kc[l].ptr,
                                                     self.vc[l].ptr, self.f16, self.ws.ptr, self.ws_bytes, s)
        except mimg.NotHandled:  # (the norm is done: the products and rope separately)
            self.qkv_rows_fused = False
            mimg.matmul_a8_quantized_group_dev(ws, self.h.ptr, T, bs if any(bs) else None, 256,
                                               [self.q.ptr, self.k.ptr, self.v.ptr], self.ws.ptr, self.ws_bytes, s)
            mimg.rope_kv_dev(self.q.ptr, self.k.ptr, self.v.ptr, pos, cidx, self.invf.ptr, T, c.heads, c.kv_heads,
                             c.head_dim, c.rope_dims, c.interleaved, self.cache_len, self.kc[l].ptr, self.vc[l].ptr,
                             self.f16, s)
        return True

    def _ffn_rows(self, l, T):
        """The FFN at 1..8 rows with 8-bit activations of blocks of 256: x
        += the attention output; h = rms_norm(x) * scale quantized (one
        launch); gate and up products with swiglu in their epilogue (one
        launch); the quantizer on the swiglu output; down. False (nothing
        launched) where the swiglu epilogue does not take the shape."""
        c, s = self.c, self.stream.handle
        p = f"blk.{l}."
        gate, up, down = (self.w[p + n] for n in ("ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"))
        F, E = c.ffn, c.embed
        fused = self.swiglu_fused if T == 1 else self.swiglu_rows_fused
        if not (self.a8 and fused and 1 <= T <= 8 and gate.dt == mimg.Q4_K and up.dt == mimg.Q4_K and
                self._block(gate) == 256 and self._block(down) in (32, 256) and gate.n == up.n == F
                and F % (4 if T == 1 else 8) == 0 and E % 256 == 0 and E <= 16384 and F <= 32768
                and p + "ffn_gate.bias" not in self.vec and p + "ffn_up.bias" not in self.vec):
            return False
        mimg.rms_norm_quant_dev(self.x.ptr, self.ao.ptr, self.vec[p + "ffn_norm.weight"].ptr, c.norm_eps, T, E,
                                self.h.ptr, 256, self.ws.ptr, self.ws_bytes, s)
        try:
            mimg.matmul_a8_quantized_swiglu_dev([gate, up], self.h.ptr, T, None, 256, self.sw.ptr, self.procs,
                                                self.ws.ptr, self.ws_bytes, s)
        except mimg.NotHandled:  # (the norm is done: the products and swiglu separately)
            if T == 1:
                self.swiglu_fused = False
            else:
                self.swiglu_rows_fused = False
            mimg.matmul_a8_quantized_group_dev([gate, up], self.h.ptr, T, None, 256, [self.g.ptr, self.u.ptr],
                                               self.ws.ptr, self.ws_bytes, s)
            mimg.swiglu_dev(self.g.ptr, self.u.ptr, self.sw.ptr, T * F, self.procs, s)
        mimg.quantize_act_dev(self.sw.ptr, T, F, self._block(down), self.ws.ptr, self.ws_bytes, s)
        mimg.matmul_a8_quantized_group_dev([down], self.sw.ptr, T, None, self._block(down), [self.ao.ptr],
                                           self.ws.ptr, self.ws_bytes, s)
        return True

    def _norm_qkv_rope(self, l, resid, qkv, qkv_b, pos, cidx):
        """At one row with 8-bit activations: the attention norm, the q/k/v
        products, rope and the cache scatter in one launch (x + resid lands in
        the other x buffer). False where that launch does not take the shape
        (nothing launched): the caller makes the separate calls."""
        if not self.a8 or not self.rope_fused or any(self._block(self.w[n]) != 256 for n in qkv):
            return False
        c, s = self.c, self.stream.handle
        p = f"blk.{l}."
        bs = [None if b is None or b not in self.vec else self.vec[b].ptr for b in qkv_b]
        try:
            mimg.rms_norm_qkv_rope_kv_dev([self.w[n] for n in qkv], self.x.ptr, resid,
                                          self.vec[p + "attn_norm.weight"].ptr, c.norm_eps, self.x_alt.ptr,
                                          bs if any(bs) else None, self.q.ptr, pos, cidx, self.invf.ptr, c.heads,
                                          c.kv_heads, c.head_dim, c.rope_dims, c.interleaved, self.cache_len,
                                          self.kc[l].ptr, self.vc[l].ptr, self.f16, s)
        except mimg.NotHandled:
            self.rope_fused = False
            return False
        self.x, self.x_alt = self.x_alt, self.x
        return True

    def _forward(self, T, ids=None, pos=None, cidx=None, kstart=None, head_rows=None):
        """Enqueues the forward pass of T rows (device arrays of token ids,
        positions, cache indices and slot starts; by default the decoder's
        own). Logits land in self.logits: all T rows, or with head_rows =
        [(row, logits row)] only those rows (the head is the largest matrix;
        generation needs the last row of each prompt only)."""
        c, s = self.c, self.stream.handle
        E, F, H, Hkv, D = c.embed, c.ffn, c.heads, c.kv_heads, c.head_dim
        ids = ids or self.ids.ptr
        pos = pos or self.pos.ptr
        cidx = cidx or self.cidx.ptr
        kstart = (kstart or self.kstart.ptr) if self.slots > 1 else None
        self.x, self.x_alt = self.x_pair  # every forward the same buffers (graphs replay them)
        mimg.embedding_dev(self.w["token_embd.weight"], ids, T, self.x.ptr, s)
        resid = None  # the previous sublayer's output, added to x by the next norm
        for l in range(c.layers):
            p = f"blk.{l}."
            qkv = [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"]
            qkv_b = [p + "attn_q.bias", p + "attn_k.bias", p + "attn_v.bias"]
            if not (T == 1 and self._norm_qkv_rope(l, resid, qkv, qkv_b, pos, cidx)) and \
                    not (4 <= T <= 8 and self._qkv_rope_rows(l, resid, qkv, qkv_b, T, pos, cidx)):
                self._norm_linears(resid, p + "attn_norm.weight", T, qkv, [self.q.ptr, self.k.ptr, self.v.ptr], qkv_b,
                                   single_fused=True)
                mimg.rope_kv_dev(self.q.ptr, self.k.ptr, self.v.ptr, pos, cidx, self.invf.ptr, T, H, Hkv, D,
                                 c.rope_dims, c.interleaved, self.cache_len, self.kc[l].ptr, self.vc[l].ptr, self.f16,
                                 s)
            mimg.attention_dev(self.q.ptr, self.kc[l].ptr, self.vc[l].ptr, cidx, kstart, T, H, Hkv, D,
                               self.cache_len, c.context, self.f16, self.o.ptr, self.att_ws.ptr, self.att_ws_bytes, s)
            self._linears([p + "attn_output.weight"], self.o.ptr, T, [self.ao.ptr])
            down = self.w[p + "ffn_down.weight"]
            if T <= 8 and self._ffn_rows(l, T):
                pass
            elif self.a8 and self._block(down) in (32, 256) and F <= 32768:
                self._norm_linears(self.ao.ptr, p + "ffn_norm.weight", T, [p + "ffn_gate.weight", p + "ffn_up.weight"],
                                   [self.g.ptr, self.u.ptr])
                # (out a buffer of its own: the refusal screen reads g and u)
                mimg.swiglu_quant_dev(self.g.ptr, self.u.ptr, self.sw.ptr, T, F, self.procs, self._block(down),
                                      self.ws.ptr, self.ws_bytes, s)
                mimg.matmul_a8_quantized_group_dev([down], self.sw.ptr, T, None, self._block(down), [self.ao.ptr],
                                                   self.ws.ptr, self.ws_bytes, s)
            else:
                self._norm_linears(self.ao.ptr, p + "ffn_norm.weight", T, [p + "ffn_gate.weight", p + "ffn_up.weight"],
                                   [self.g.ptr, self.u.ptr])
                mimg.swiglu_dev(self.g.ptr, self.u.ptr, self.g.ptr, T * F, self.procs, s)
                self._linears([p + "ffn_down.weight"], self.g.ptr, T, [self.ao.ptr])
            resid = self.ao.ptr
        V = self.vocab
        if head_rows is None and self.a8 and E <= 32768:
            block = self._block(self.head)
            mimg.rms_norm_quant_dev(self.x.ptr, resid, self.vec["output_norm.weight"].ptr, c.norm_eps, T, E,
                                    self.h.ptr, block, self.ws.ptr, self.ws_bytes, s)
            mimg.matmul_a8_quantized_group_dev([self.head], self.h.ptr, T, None, block, [self.logits.ptr], self.ws.ptr,
                                               self.ws_bytes, s)
            return
        mimg.rms_norm_dev(self.x.ptr, resid, self.vec["output_norm.weight"].ptr, c.norm_eps, T, E, self.h.ptr, s)
        for src, dst, n in ([(0, 0, T)] if head_rows is None else [(r, d, 1) for r, d in head_rows]):
            xh, yh = self.h.ptr + src * E * 4, self.logits.ptr + dst * V * 4
            if self.a8:
                mimg.linear_a8_dev(self.head, xh, n, None, self._block(self.head), yh, self.ws.ptr, self.ws_bytes, s)
            elif 0 < self.f32_tile_rows <= n:
                mimg.linear_f32_mfma_dev(self.head, xh, n, None, yh, s)
            else:
                mimg.linear_f32_dev(self.head, xh, n, None, yh, s)

    def _set_rows(self, tokens, positions, slots=None):
        tokens = np.asarray(tokens, np.int32).ravel()
        positions = np.asarray(positions, np.int64).ravel()
        T = tokens.size
        if T == 0 or T > self.R or positions.size != T:
            raise ValueError(f"{T} tokens with {positions.size} positions (1..{self.R})")
        slots = np.zeros(T, np.int64) if slots is None else np.asarray(slots, np.int64).ravel()
        if slots.size != T or slots.min() < 0 or slots.max() >= self.slots:
            raise ValueError(f"slots {slots} (0..{self.slots - 1})")
        if positions.min() < 0 or positions.max() >= self.c.context:
            raise ValueError(f"positions outside 0..{self.c.context - 1}")
        start = slots * self.c.context
        self.stream.sync()
        self.ids.upload(tokens)
        self.pos.upload(positions)
        self.cidx.upload(start + positions)
        self.kstart.upload(start)
        return T

    # ---- API -----------------------------------------------------------------

    def forward(self, tokens, positions, slots=None):
        """Logits [T, vocab] (host) for the tokens at the positions; the
        cache is updated (reference Session.Step)."""
        T = self._set_rows(tokens, positions, slots)
        self._forward(T)
        self.stream.sync()
        return self.logits.download(np.float32, T * self.vocab).reshape(T, self.vocab)

    def _decode_step(self, n):
        """One greedy step of n sequences: forward of the tokens in ids,
        pick, append, advance."""
        self._forward(n)
        mimg.argmax_dev(self.logits.ptr, n, self.vocab, self.chosen.ptr, self.stream.handle)
        mimg.greedy_advance_dev(self.chosen.ptr, self.ids.ptr, self.pos.ptr, self.cidx.ptr, self.out.ptr,
                                self.count.ptr, self.out_cap, n, self.stream.handle)

    def _decode_graph(self, n):
        g = self.graphs.get(n)
        if g is None:
            g = self.graphs[n] = hiprt.Graph(self.stream, lambda: self._decode_step(n))
        return g

    def _ensure_out(self, cap, n):
        if self.out is None or self.out_cap < cap or self.out.nbytes < cap * n * 4:
            self.stream.sync()
            for g in self.graphs.values():  # captured with the old buffer
                g.destroy()
            self.graphs = {}
            self.out = hiprt.DeviceBuffer(cap * n * 4)
            self.out_cap = cap

    def generate(self, prompts, n_new, slots=None, graph=True, timing=None):
        """Greedy continuation of each prompt (one per slot, all of the same
        length): n_new tokens each, [len(prompts), n_new] (reference
        cmd/mim-run/main.go generate). The prompt rows run in batches of at
        most max_rows, the first pick is made on the device, and every
        decode step is one graph replay. With a dict as timing, it receives
        the device times of the prompt (to the first pick) and of the
        decode steps."""
        prompts = np.atleast_2d(np.asarray(prompts, np.int32))
        n, P = prompts.shape
        if n > self.slots or n > self.R:
            raise ValueError(f"{n} prompts, {self.slots} slots, {self.R} rows")
        if P < 1 or P + n_new - 1 > self.c.context:
            raise ValueError(f"{P} + {n_new} tokens exceed the context {self.c.context}")
        slots = np.arange(n, dtype=np.int64) if slots is None else np.asarray(slots, np.int64)
        if slots.size != n or slots.min() < 0 or slots.max() >= self.slots:
            raise ValueError(f"slots {slots}")
        self._ensure_out(max(n_new, 1), n)
        s = self.stream.handle
        C = self.c.context
        # every prompt row's inputs, and the state of the first decode step
        B = hiprt.DeviceBuffer
        rows_pos = np.tile(np.arange(P, dtype=np.int64), n)
        rows_start = np.repeat(slots * C, P)
        p_ids, p_pos = B.from_array(prompts.ravel()), B.from_array(rows_pos)
        p_cidx, p_start = B.from_array(rows_start + rows_pos), B.from_array(rows_start)
        self.stream.sync()
        self.pos.upload(np.full(n, P - 1, np.int64))
        self.cidx.upload(slots * C + P - 1)
        self.kstart.upload(slots * C)
        self.count.upload(np.zeros(1, np.int32))
        ev = [hiprt.Event() for _ in range(3)]
        ev[0].record(self.stream)
        for c0 in range(0, n * P, self.R):
            T = min(self.R, n * P - c0)
            heads = [(i * P + P - 1 - c0, i) for i in range(n) if c0 <= i * P + P - 1 < c0 + T]
            self._forward(T, p_ids.ptr + 4 * c0, p_pos.ptr + 8 * c0, p_cidx.ptr + 8 * c0, p_start.ptr + 8 * c0,
                          head_rows=heads)
        mimg.argmax_dev(self.logits.ptr, n, self.vocab, self.chosen.ptr, s)
        mimg.greedy_advance_dev(self.chosen.ptr, self.ids.ptr, self.pos.ptr, self.cidx.ptr, self.out.ptr,
                                self.count.ptr, self.out_cap, n, s)
        ev[1].record(self.stream)
        if graph and n_new > 1:
            g = self._decode_graph(n)
            for _ in range(n_new - 1):
                g.launch(self.stream)
        else:
            for _ in range(n_new - 1):
                self._decode_step(n)
        ev[2].record(self.stream)
        self.stream.sync()
        if timing is not None:
            timing["prompt_ms"] = ev[0].elapsed_ms(ev[1])
            timing["decode_ms"] = ev[1].elapsed_ms(ev[2])
            timing["prompt_rows"], timing["decode_steps"] = n * P, n_new - 1
        return self.out.download(np.int32, n_new * n).reshape(n_new, n).T.copy()

    def reset(self):
        """Clears the cache (a new session)."""
        self.stream.sync()
        for buf in self.kc + self.vc:
            buf.zero()
