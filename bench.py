#!/usr/bin/env python3
"""Benchmark of the block-quantized linear-layer path on one MI355X.

Workload: the seven linear layers of one
Llama-3-8B-shaped decoder layer at batch M = 1, Q4_K_M mixture
  q 4096->4096 Q4_K, k 4096->1024 Q4_K, v 4096->1024 Q6_K, o 4096->4096 Q4_K,
  gate/up 4096->14336 Q4_K, down 14336->4096 Q6_K,
run as dequant_matmul_a8.v2 with activation blocks of 256 (the path
mim-import writes for K-quant weights): each step quantizes the layer's four
input vectors (attention input, attention output, FFN input, FFN hidden) and
runs the seven products. Weights W ~ N(0, 0.02^2) (numpy PCG64, seeds 0..6 in
the order above), encoded on the GPU by libmimg's encoder; activations
x ~ N(0, 1) (seeds 100..103). Synthetic data; no checkpoint.

The four inputs are independent, so at one row the step (--step set, the
default) quantizes them in one launch and runs the seven products in one
launch (mimg_linear_a8_set_dev, bit for bit the separate calls). The same
layer set as a decoder layer calls it, one launch per grouped call (q/k/v,
o, gate/up, down: --step group), is timed beside it and reported under
config.other_forms_us_per_step; a decoder layer's calls depend on each
other, and the decode section below runs them that way.

To measure HBM rather than the 256 MB MALL, the weights are copied into
--rotate (default 32) distinct layers (4.4 GB, a whole 8B model's linears)
and step s uses layer s mod rotate. The steps over the 32 layers (one
token's linear sets) are captured in one HIP graph (--graph-steps). Timed
region: exactly --steps steps between two synchronisations.

value = bytes per step / time per step, bytes = the sum of
N*(K/QK)*block_bytes + K*4 + N*4 over the seven matrices (the benchmark's
published formula for this metric).

roofline: the step's longest launch, at one row the set's product launch
(the seven matrices, 139 MB), timed alone (graphs of --rotate launches over
the rotation copies, HIP events on the launch stream), its algorithmic bytes
over that time against 8 TB/s; traffic from the committed rocprofv3
FETCH/WRITE summary; the read ceiling: a plain streaming read of the same
weight bytes in one launch, timed the same way. The grouped gate+up launch
(the roofline kernel of the grouped form), gate alone and the Q6_K down
launch are reported beside it.

cfg0: the single 4096 x 4096 Q4_K product of one
activation row, quantized inside the launch, per call.

prefill: the gate and down products at M = 64, 512, 2048
activation rows on the int8 matrix-core GEMMs (Q4_K/Q6_K with activation
blocks of 256; Q8_0 with blocks of 32) and with float32 activations on the
fp32 matrix cores. --prefill-only times only these and prints them as one
JSON line (with --eager, launch by launch: the form profiler runs use).

cpu_baseline: the oracle's C restatement of the one-row product
(oracle/mimref.c, AVX2, threaded over weight rows) on the host's cores, on
a bounded sample of the cfg1 layer set.

The "decode" section runs whole greedy generation on the GPU decoder
(mimir-model_amd/decoder.py) with random Q4_K_M weights of two model shapes
(BASELINE.json configs[3] and [4]): a Llama-3.2-1B shape with a 32-token
prompt (uniform ids, seed 7) and 128 new tokens, and a Llama-3-8B shape
with a 512-token prompt and 256 new tokens at batch 1 and at batch 8 (eight
sequences in eight cache slots), f16 key-value cache. Reported: decode
tokens/s (every sequence's new tokens over the device time of the decode
steps), prompt tokens/s, and the weight bytes a decode step reads over the
step time. Unless --no-cpu, the CPU restatement (oracle/llama_ref.py) decodes
the first tokens of each shape from the same weights and its ids are
compared with the GPU's (8 tokens; the 8B shape on a 32-token prompt).
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mimir-model_amd"))

import hiprt  # noqa: E402
import mimg  # noqa: E402

METRIC = "Q4_K GEMV GB/s (% of HBM peak); decode tok/s at 8B Q4_K_M; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
Q4_K, Q6_K = mimg.Q4_K, mimg.Q6_K

# (name, N, K, dtype, weight seed, input index)
CFG1 = [
    ("q", 4096, 4096, Q4_K, 0, 0),
    ("k", 1024, 4096, Q4_K, 1, 0),
    ("v", 1024, 4096, Q6_K, 2, 0),
    ("o", 4096, 4096, Q4_K, 3, 1),
    ("gate", 14336, 4096, Q4_K, 4, 2),
    ("up", 14336, 4096, Q4_K, 5, 2),
    ("down", 4096, 14336, Q6_K, 6, 3),
]
INPUT_K = [4096, 4096, 4096, 14336]


def weight_bytes(n, k, dt):
    return n * (k // 256) * (144 if dt == Q4_K else 210)


def step_bytes(rows=1):
    return sum(weight_bytes(n, k, dt) + rows * (k * 4 + n * 4) for _, n, k, dt, _, _ in CFG1)


def launch_bytes(n, k, dt, rows=1):
    """Algorithmic bytes of one GEMV launch: the weight blocks, and per
    activation row the int8 quants, one f32 scale per 256, the per-32 (Q4_K)
    or per-16 (Q6_K) int16 sums, and the f32 outputs."""
    sums = (k // 32) * 2 if dt == Q4_K else (k // 16) * 2
    return weight_bytes(n, k, dt) + rows * (k + (k // 256) * 4 + sums + n * 4)


def make_weights(stream, rotate, log):
    """Encodes the seven matrices on the GPU and registers `rotate` device
    copies of each. Returns ([per layer: {name: Weight}], {name: host bytes})."""
    layers = [dict() for _ in range(rotate)]
    host_bytes = {}
    for name, n, k, dt, seed, _ in CFG1:
        t0 = time.time()
        w32 = np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32)
        w32 *= np.float32(0.02)
        xd = hiprt.DeviceBuffer.from_array(w32)
        del w32
        nb = weight_bytes(n, k, dt)
        enc = hiprt.DeviceBuffer(nb)
        mimg.quantize_dev(dt, xd.ptr, n * k, enc.ptr, nb, stream.handle)
        stream.sync()
        xd.free()
        host_bytes[name] = enc.download(np.uint8)
        for l in range(rotate):
            layers[l][name] = mimg.Weight((enc.ptr, nb), dt, n, k, device=True)
        enc.free()
        log(f"  {name}: {n}x{k} {'Q4_K' if dt == Q4_K else 'Q6_K'} {nb / 1e6:.1f} MB x {rotate} ({time.time() - t0:.1f} s)")
    return layers, host_bytes


def make_q8_0_weights(stream, rotate, log):
    """BASELINE configs[2]'s Q8_0 variant of gate (= up's shape) and down:
    the same f32 weights (seeds 4 and 6) encoded as Q8_0 (the reference's
    encoder, mim.Quantize), `rotate` device copies each."""
    layers = [dict() for _ in range(rotate)]
    for name, n, k, _, seed, _ in CFG1:
        if name not in ("gate", "down"):
            continue
        t0 = time.time()
        w32 = np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32)
        w32 *= np.float32(0.02)
        xd = hiprt.DeviceBuffer.from_array(w32)
        del w32
        nb = n * (k // 32) * 34
        enc = hiprt.DeviceBuffer(nb)
        mimg.quantize_dev(mimg.Q8_0, xd.ptr, n * k, enc.ptr, nb, stream.handle)
        stream.sync()
        xd.free()
        for l in range(rotate):
            layers[l][name] = mimg.Weight((enc.ptr, nb), mimg.Q8_0, n, k, device=True)
        enc.free()
        log(f"  {name} Q8_0: {n}x{k} {nb / 1e6:.1f} MB x {rotate} ({time.time() - t0:.1f} s)")
    return layers


def cpu_baseline(host_bytes, xs, seconds, log):
    """The oracle's linear_a8 (C restatement of the reference numerics) over
    the seven matrices of one layer, on this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import mimref

    threads = min(16, os.cpu_count() or 1)
    nbytes = step_bytes(xs[0].shape[0])

    def one_layer(t):
        for name, n, k, dt, _, inp in CFG1:
            mimref.linear_a8(xs[inp], host_bytes[name], dt, n, k, block=256, threads=t)

    one_layer(threads)  # warm the page cache
    reps, t0 = 0, time.time()
    while time.time() - t0 < seconds or reps == 0:
        one_layer(threads)
        reps += 1
    all_s = (time.time() - t0) / reps
    t0 = time.time()
    one_layer(1)
    one_s = time.time() - t0
    cpu_model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    log(f"  cpu: {threads} threads {nbytes / all_s / 1e9:.2f} GB/s, 1 thread {nbytes / one_s / 1e9:.2f} GB/s")
    return {
        "value": round(nbytes / all_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"one cfg1 layer set (7 matrices, {nbytes / 1e6:.1f} MB) at M=1 through oracle/ linear_a8 "
                  f"(C restatement of dotQ4KQ8KAVX2/dotQ6KQ8KAVX2 numerics), {reps} passes in {reps * all_s:.1f} s",
        "value_1thread": round(nbytes / one_s / 1e9, 3),
        "cpu_model": cpu_model,
        "nproc": os.cpu_count(),
    }


def decode_cpu_check(cfg, tensors, prompt, gpu_ids, n, log):
    """The CPU restatement of the decoder (oracle/llama_ref.py, the linears
    through the C oracle on this host's cores) on the same weight bytes and
    prompt: its first n greedy ids, compared with the GPU's, and its decode
    rate (tokens/s after the prompt)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import llama_ref
    import synthetic

    threads = min(16, os.cpu_count() or 1)
    ref = llama_ref.Decoder(llama_ref.Model(cfg, synthetic.host_bytes(tensors)), a8=True, cache_f16=True,
                            threads=threads)
    P = len(prompt)
    t0 = time.time()
    lg = ref.forward(prompt, np.arange(P))[-1]
    t_prompt = time.time() - t0
    ids = []
    t0 = time.time()
    for i in range(n):
        ids.append(llama_ref.argmax(lg))
        if i + 1 < n:
            lg = ref.forward([ids[-1]], [P + i])[0]
    t_dec = time.time() - t0
    match = ids == [int(v) for v in gpu_ids[:n]]
    log(f"  cpu restatement: {n} ids {'==' if match else '!='} GPU; {(n - 1) / t_dec:.2f} tok/s decode, "
        f"{P / t_prompt:.1f} tok/s prompt ({threads} threads)")
    return {"ids_equal_gpu": match, "tokens_checked": n, "decode_tok_per_s": round((n - 1) / t_dec, 3),
            "prompt_tok_per_s": round(P / t_prompt, 2), "cores": threads, "kind": "port"}


def cfg4_oracle_check(tensors, prompt, gpu_ids, log):
    """The batch-1 8B run against tests/golden/cfg4_ids.json: the CPU
    restatement's first 32 greedy ids for the same weights (checked by their
    digests) and the same 512-token prompt."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_cfg4_ids as mk
    import synthetic

    with open(mk.FIXTURE) as f:
        fx = json.load(f)
    same_weights = mk.digests(synthetic.host_bytes({n: tensors[n] for n in mk.DIGESTED})) == fx["weights_sha256"]
    same_prompt = np.array_equal(prompt, mk.prompts(synthetic.LLAMA_8B["vocab"])[0])
    n = min(len(fx["ids"]), len(gpu_ids))
    equal = same_weights and same_prompt and [int(v) for v in gpu_ids[:n]] == fx["ids"][:n]
    log(f"  llama8b 512-token prompt: first {n} GPU ids {'==' if equal else '!='} the CPU restatement's "
        f"(fixture; weights {'match' if same_weights else 'differ'})")
    return {"ids_equal_cpu_restatement": bool(equal), "tokens_checked": n, "weights_match_fixture": bool(same_weights),
            "fixture": "tests/golden/cfg4_ids.json"}


def decode_bench(name, log, graph=True, cpu=False, batches=(1, 8), new_tokens=None):
    """Greedy generation on the GPU decoder with a random model of the
    named shape (module docstring); batches selects the 8B runs."""
    import decoder
    import synthetic

    cfg = dict(synthetic.LLAMA_1B if name == "llama1b" else synthetic.LLAMA_8B)
    runs = [(32, 128, 1)] if name == "llama1b" else [(512, 256, b) for b in batches]
    if new_tokens:  # profiler runs: fewer decode steps
        runs = [(p, new_tokens, b) for p, _, b in runs]
    cfg["context"] = max(p + n for p, n, _ in runs)
    t0 = time.time()
    # the 8B weights are the GPU tests' (seed 3), whose 512-token prompt ids
    # the CPU restatement wrote into tests/golden/cfg4_ids.json
    tensors = synthetic.build(cfg, seed=1 if name == "llama1b" else 3, log=log)
    slots = max(b for _, _, b in runs)
    rows = max(min(p * b, 512) for p, _, b in runs)
    dec = decoder.Decoder(cfg, tensors, a8=True, cache_f16=True, max_rows=rows, slots=slots)
    log(f"  {name}: model and decoder ready in {time.time() - t0:.1f} s")
    step_bytes_tok = synthetic.weight_bytes(cfg, per_token=True)
    out = {}
    for P, n_new, batch in runs:
        prompts = np.random.default_rng(7).integers(0, cfg["vocab"], (batch, P)).astype(np.int32)
        dec.generate(prompts, 4, graph=graph)  # warm up: captures the decode graph
        dec.reset()
        tm = {}
        ids = dec.generate(prompts, n_new, timing=tm, graph=graph)
        dec.reset()
        step_ms = tm["decode_ms"] / tm["decode_steps"]
        key = f"{name}_P{P}_N{n_new}_B{batch}"
        out[key] = {
            "decode_tok_per_s": round(batch * tm["decode_steps"] / (tm["decode_ms"] * 1e-3), 1),
            "ms_per_step": round(step_ms, 4),
            "prompt_tok_per_s": round(tm["prompt_rows"] / (tm["prompt_ms"] * 1e-3), 1),
            "prompt_ms": round(tm["prompt_ms"], 3),
            "weight_GB_per_s": round(step_bytes_tok / (step_ms * 1e-3) / 1e9, 1),
            "weight_bytes_per_step": step_bytes_tok,
            "first_ids": ids[0, :8].tolist(),
            "graphs": graph,
        }
        if cpu and batch == 1 and name == "llama1b":
            out[key]["cpu_restatement"] = decode_cpu_check(cfg, tensors, prompts[0], ids[0], 8, log)
        if batch == 1:
            b1_ids = ids[0]
            if name == "llama8b" and P == 512:
                out[key]["oracle_ids"] = cfg4_oracle_check(tensors, prompts[0], ids[0], log)
        elif P == runs[0][0] and runs[0][2] == 1:
            # slot 0 holds the batch-1 run's prompt: the same ids
            out[key]["slot0_ids_equal_batch1"] = bool(np.array_equal(ids[0], b1_ids))
        log(f"  {key}: {out[key]}")
    if cpu and name == "llama8b":
        # The 512-token prompt is too long for the CPU restatement within the
        # bench's budget: a 32-token prompt (seed 7) and 8 greedy ids on both.
        short = np.random.default_rng(7).integers(0, cfg["vocab"], (1, 32)).astype(np.int32)
        dec.reset()
        gids = dec.generate(short, 8, graph=graph)
        dec.reset()
        out["llama8b_P32_N8_B1_cpu_check"] = {"cpu_restatement": decode_cpu_check(cfg, tensors, short[0], gids[0], 8,
                                                                                   log)}
    del dec
    tensors.clear()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--rotate", type=int, default=32)
    ap.add_argument("--rows", type=int, default=1, help="activation rows M (1 = cfg1; 8 = cfg4's batch 8)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch without HIP graphs (every timed section)")
    ap.add_argument("--prefill-rows", default="64,512,2048",
                    help="activation rows of the prefill GEMM measurements (comma list; empty to skip)")
    ap.add_argument("--prefill-kinds", default="a8,q8_0,b32,f32",
                    help="prefill products to time: a8 (Q4_K/Q6_K x 8-bit blocks of 256), q8_0 (Q8_0 x 8-bit), "
                         "b32 (Q4_K/Q6_K x 8-bit blocks of 32, the tiled opt-in), f32")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the prefill products (for profiler runs) and print them as one JSON line")
    ap.add_argument("--decode-batches", default="1,8", help="batch sizes of the llama8b decode runs")
    ap.add_argument("--decode-tokens", type=int, default=0,
                    help="new tokens per decode run (default: the configs' 128 and 256; fewer for profiler runs)")
    ap.add_argument("--decode", default="llama1b,llama8b",
                    help="whole-model decode runs (comma list of llama1b, llama8b; empty to skip)")
    ap.add_argument("--step", default="", choices=["", "chain", "group", "set"],
                    help="set (default at one row): the four groups' independent inputs quantized in one launch and "
                         "the seven products in one launch (mimg_linear_a8_set_dev); group (default at more rows): "
                         "one launch per grouped call, as a decoder layer makes them; chain: the four grouped "
                         "products as one chain launch (mimg_linear_a8_chain_dev, one row only)")
    ap.add_argument("--graph-steps", type=int, default=0,
                    help="steps captured in one HIP graph (consecutive rotation layers; divides --rotate; "
                         "default: --rotate)")
    ap.add_argument("--roofline-replays", type=int, default=8,
                    help="replays of the graph of --rotate single-kernel launches timed for the roofline")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (row sharding is a design note). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    mimg.init(0)
    stream = hiprt.Stream()
    M = args.rows
    log(f"bench: cfg1 layer set, M={M}, rotate {args.rotate}")
    layers, host_bytes = make_weights(stream, args.rotate, log)

    xs = [np.random.default_rng(100 + i).standard_normal((M, k), dtype=np.float32) for i, k in enumerate(INPUT_K)]
    xd = [hiprt.DeviceBuffer.from_array(x) for x in xs]
    ws_bytes = [mimg.a8_workspace_bytes(M, k) for k in INPUT_K]
    ws = [hiprt.DeviceBuffer(b) for b in ws_bytes]
    yd = {name: hiprt.DeviceBuffer(M * n * 4) for name, n, _, _, _, _ in CFG1}

    # Prefill: the gate (Q4_K) and down (Q6_K) products
    # at M activation rows on the int8 MFMA GEMM, activations quantized
    # beforehand; a graph of --rotate launches over the rotation copies
    # (with --eager the same launches issued directly). Ops = 2*M*N*K; the fraction is of MI355X's dense int8 peak.
    # With f32 (BASELINE.json north_star's f32-activation prefill,
    # dequant_matmul.v1): the same products with float32 activations on the
    # fp32 matrix cores (mimg_linear_f32_mfma_dev), fraction of the dense
    # fp32 matrix peak.
    def prefill(name, rows, f32=False, q8_layers=None, b32=False):
        _, n, k, dt, _, _ = next(c for c in CFG1 if c[0] == name)
        block = 32 if (q8_layers or b32) else 256
        xp = hiprt.DeviceBuffer.from_array(np.random.default_rng(200 + rows).standard_normal((rows, k), dtype=np.float32))
        wsb = mimg.a8_workspace_bytes(rows, k)
        wsp = hiprt.DeviceBuffer(wsb)
        yp = hiprt.DeviceBuffer(rows * n * 4)
        mimg.quantize_act_dev(xp.ptr, rows, k, block, wsp.ptr, wsb, stream.handle)
        src = q8_layers or layers

        def launches():
            for l in range(args.rotate):
                if f32:
                    mimg.linear_f32_mfma_dev(src[l][name], xp.ptr, rows, None, yp.ptr, stream.handle)
                elif q8_layers:
                    mimg.matmul_a8_quantized_q8_0_tiled_dev(src[l][name], xp.ptr, rows, None, yp.ptr, wsp.ptr, wsb,
                                                            stream.handle)
                elif b32:
                    mimg.matmul_a8_quantized_b32_tiled_dev(src[l][name], xp.ptr, rows, None, yp.ptr, wsp.ptr, wsb,
                                                           stream.handle)
                else:
                    mimg.matmul_a8_quantized_dev(src[l][name], xp.ptr, rows, None, block, yp.ptr, wsp.ptr, wsb,
                                                 stream.handle)

        a, b = hiprt.Event(), hiprt.Event()
        if args.eager:
            launches()
            a.record(stream)
            launches()
            b.record(stream)
            b.sync()
        else:
            g = hiprt.Graph(stream, launches)
            g.launch(stream)
            a.record(stream)
            g.launch(stream)
            b.record(stream)
            b.sync()
            g.destroy()
        us = a.elapsed_ms(b) * 1e3 / args.rotate
        for buf in (xp, wsp, yp):
            buf.free()
        tops = 2.0 * rows * n * k / (us * 1e-6) / 1e12
        if f32:
            return {"us_per_launch": round(us, 2), "TFLOP_per_s": round(tops, 1),
                    "frac_fp32_peak": round(tops / FP32_PEAK_TFLOPS, 4)}
        return {"us_per_launch": round(us, 2), "TOP_per_s": round(tops, 1),
                "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}

    def run_prefills():
        prefill_res, prefill_q8, prefill_f32 = {}, {}, {}
        prefill_b32.clear()
        prefill_rows = [int(r) for r in args.prefill_rows.split(",") if r]
        q8_layers = make_q8_0_weights(stream, args.rotate, log) if prefill_rows and "q8_0" in kinds else None
        for rows in prefill_rows:
            for name in ("gate", "down"):
                if "a8" in kinds:
                    prefill_res[f"{name}_M{rows}"] = prefill(name, rows)
                    log(f"  prefill {name} M={rows}: {prefill_res[f'{name}_M{rows}']}")
                if q8_layers:
                    prefill_q8[f"{name}_M{rows}"] = prefill(name, rows, q8_layers=q8_layers)
                    log(f"  prefill Q8_0 {name} M={rows}: {prefill_q8[f'{name}_M{rows}']}")
                if "b32" in kinds:
                    prefill_b32[f"{name}_M{rows}"] = prefill(name, rows, b32=True)
                    log(f"  prefill {name} blocks of 32 M={rows}: {prefill_b32[f'{name}_M{rows}']}")
                if "f32" in kinds:
                    prefill_f32[f"{name}_M{rows}"] = prefill(name, rows, f32=True)
                    log(f"  prefill f32 {name} M={rows}: {prefill_f32[f'{name}_M{rows}']}")
        if q8_layers:
            q8_layers.clear()
        return prefill_res, prefill_q8, prefill_f32

    kinds = args.prefill_kinds.split(",")
    prefill_b32 = {}
    if args.prefill_only:
        pr, pq, pf = run_prefills()
        print(json.dumps({"prefill": pr, "prefill_q8_0": pq, "prefill_kquant_b32": prefill_b32, "prefill_f32": pf,
                          "graphs": not args.eager}), flush=True)
        return

    # A decoder layer's calls: q, k and v share the attention input and gate
    # and up the FFN input, so each pair/triple is one grouped call
    # (dequant_matmul_a8.v2 each, bit for bit); o and down have inputs of
    # their own.
    groups = [[c for c in CFG1 if c[5] == i] for i in range(len(INPUT_K))]

    step_kind = args.step or ("set" if M == 1 else "group")
    if step_kind in ("chain", "set") and M != 1:
        raise SystemExit("--step chain and --step set run one activation row (--rows 1)")

    def set_groups(l):
        return [([layers[l][c[0]] for c in grp], xd[i].ptr, None, [yd[c[0]].ptr for c in grp])
                for i, grp in enumerate(groups)]

    set_ws_bytes = mimg.linear_a8_set_workspace_bytes(set_groups(0)) if M == 1 else 0
    set_ws = hiprt.DeviceBuffer(set_ws_bytes) if M == 1 else None
    sync_bytes = mimg.chain_sync_bytes()
    sync = hiprt.DeviceBuffer(sync_bytes)
    mimg.chain_sync_init(sync.ptr, sync_bytes, stream.handle)

    def enqueue_step(kind, l):
        if kind == "set":
            # the seven products' independent inputs quantized in one launch,
            # the products in one launch
            mimg.linear_a8_set_dev(set_groups(l), set_ws.ptr, set_ws_bytes, stream.handle)
        elif kind == "chain":
            # the layer set as one launch: four phases, each phase's weights
            # streamed without a break after the one before
            mimg.linear_a8_chain_dev([([layers[l][c[0]] for c in grp], xd[i].ptr, None, [yd[c[0]].ptr for c in grp])
                                      for i, grp in enumerate(groups)], sync.ptr, sync_bytes, stream.handle)
        else:
            for i, grp in enumerate(groups):
                mimg.linear_a8_group_dev([layers[l][c[0]] for c in grp], xd[i].ptr, M, None, 256,
                                         [yd[c[0]].ptr for c in grp], ws[i].ptr, ws_bytes[i], stream.handle)

    # A graph holds gs consecutive steps (layers l .. l+gs-1 of the rotation:
    # by default all 32, one token's linear sets, as a decode step's graph
    # holds all of a token's layers); with gs = 1 the host launches one graph
    # per step.
    gs = args.graph_steps or args.rotate
    if args.rotate % gs or args.steps % gs or args.warmup % gs:
        raise SystemExit("--graph-steps must divide --rotate, --steps and --warmup")
    if args.eager:
        gs = 1

    def time_steps(kind):
        """Warm-up, then exactly --steps steps of `kind` between two events
        on the launch stream (and device synchronisations); us per step and
        the wall time per step."""
        graphs = []
        if args.eager:
            def run(l):
                enqueue_step(kind, l)
        else:
            def enqueue_steps(l0):
                for l in range(l0, l0 + gs):
                    enqueue_step(kind, l)

            graphs = [hiprt.Graph(stream, lambda l0=l0: enqueue_steps(l0)) for l0 in range(0, args.rotate, gs)]

            def run(l):
                graphs[l // gs].launch(stream)

        for s in range(0, args.warmup, gs):
            run(s % args.rotate)
        stream.sync()
        e0, e1 = hiprt.Event(), hiprt.Event()
        hiprt.device_sync()
        t0 = time.perf_counter()
        e0.record(stream)
        for s in range(0, args.steps, gs):
            run(s % args.rotate)
        e1.record(stream)
        e1.sync()
        hiprt.device_sync()
        wall = time.perf_counter() - t0
        us = e0.elapsed_ms(e1) * 1e3 / args.steps
        for g in graphs:
            g.destroy()
        if kind == "chain":
            st = mimg.chain_status(sync.ptr)
            if st:
                raise SystemExit(f"chain status {st}: a device barrier wait timed out")
        log(f"  timed ({kind}, {gs} steps a graph): {args.steps} steps, {us:.2f} us/step (events), "
            f"wall {wall * 1e6 / args.steps:.2f} us/step, {step_bytes(M) / (us * 1e-6) / 1e9:.1f} GB/s")
        return us

    step_us = time_steps(step_kind)
    ms_per_step = step_us * 1e-3
    value = step_bytes(M) / (ms_per_step * 1e-3) / 1e9
    # the same layer set as a decoder layer calls it (one launch per grouped
    # call), timed the same way beside the headline form
    other_us = {k: round(time_steps(k), 3) for k in ("group", "set") if k != step_kind and (k == "group" or M == 1)}

    # Roofline of the dominant kernel of the step: the Q4_K GEMV launch that
    # computes gate and up together (2 x 14336 x 4096, 66 MB; the step's
    # grouped call), per-launch HIP events on the launch stream, over
    # distinct rotation copies so every launch reads from HBM. The same
    # kernel on gate alone and the Q6_K down launch are reported beside it.
    def per_launch(names):
        """The GEMV kernel alone on one matrix: activations quantized once
        beforehand, then a HIP graph of `rotate` back-to-back launches of the
        pair kernel (one per rotation copy, so every launch reads its
        weights from HBM), replayed --roofline-replays times between two
        events on the launch stream. Returns the average time per launch
        (graph time / launches, so the small gaps between kernels are
        included), the algorithmic bytes per launch and their rate."""
        cs = [next(c for c in CFG1 if c[0] == name) for name in names]
        _, n, k, dt, _, inp = cs[0]
        mimg.quantize_act_dev(xd[inp].ptr, M, k, 256, ws[inp].ptr, ws_bytes[inp], stream.handle)

        def launches():
            for l in range(args.rotate):
                mimg.matmul_a8_quantized_group_dev([layers[l][name] for name in names], xd[inp].ptr, M, None, 256,
                                                   [yd[name].ptr for name in names], ws[inp].ptr, ws_bytes[inp],
                                                   stream.handle)

        g = hiprt.Graph(stream, launches)
        for _ in range(2):
            g.launch(stream)
        a, b = hiprt.Event(), hiprt.Event()
        a.record(stream)
        for _ in range(args.roofline_replays):
            g.launch(stream)
        b.record(stream)
        b.sync()
        us = a.elapsed_ms(b) * 1e3 / (args.roofline_replays * args.rotate)
        # the activation row is read once per launch; weights and outputs per matrix
        nbytes = sum(launch_bytes(c[1], c[2], c[3], M) for c in cs) - (len(cs) - 1) * (launch_bytes(0, k, dt, M))
        return us, nbytes, nbytes / (us * 1e-6) / 1e9

    r_us, r_bytes, r_gbs = per_launch(["gate", "up"])
    g_us, g_bytes, g_gbs = per_launch(["gate"])
    d_us, d_bytes, d_gbs = per_launch(["down"])

    def set_launch_bytes():
        """Algorithmic bytes of the set's product launch: every matrix's
        weight blocks and outputs, and each group's quantized row once (int8
        quants, one f32 scale per 256, the per-32 sums if a Q4_K matrix reads
        it, the per-16 sums if a Q6_K one does)."""
        total = 0
        for grp in groups:
            k = grp[0][2]
            total += k + (k // 256) * 4
            total += (k // 32) * 2 if any(c[3] == Q4_K for c in grp) else 0
            total += (k // 16) * 2 if any(c[3] == Q6_K for c in grp) else 0
            total += sum(weight_bytes(c[1], c[2], c[3]) + c[1] * 4 for c in grp)
        return total

    def set_per_launch():
        """The set's product launch alone (mimg_matmul_a8_quantized_set_dev):
        the four rows quantized once by a set call, then a HIP graph of
        `rotate` product launches over the rotation copies, replayed
        --roofline-replays times between two events on the launch stream."""
        mimg.linear_a8_set_dev(set_groups(0), set_ws.ptr, set_ws_bytes, stream.handle)

        def launches():
            for l in range(args.rotate):
                mimg.matmul_a8_quantized_set_dev(set_groups(l), set_ws.ptr, set_ws_bytes, stream.handle)

        g = hiprt.Graph(stream, launches)
        for _ in range(2):
            g.launch(stream)
        a, b = hiprt.Event(), hiprt.Event()
        a.record(stream)
        for _ in range(args.roofline_replays):
            g.launch(stream)
        b.record(stream)
        b.sync()
        g.destroy()
        us = a.elapsed_ms(b) * 1e3 / (args.roofline_replays * args.rotate)
        nbytes = set_launch_bytes()
        return us, nbytes, nbytes / (us * 1e-6) / 1e9

    use_set_roof = step_kind == "set"
    if use_set_roof:
        s_us, s_bytes, s_gbs = set_per_launch()
        log(f"  set product launch (the seven matrices, {s_bytes} B): {s_us:.2f} us/launch, {s_gbs:.0f} GB/s")

    # The read ceiling of the roofline launch, measured here: a plain
    # streaming read (mimg_stream_read_dev: 16-byte nontemporal loads, every
    # load of a thread in flight at once, nothing computed) of the same
    # gate and up bytes in one launch, timed the same way over the rotation
    # copies; the best of three workgroup sizes.
    sink = hiprt.DeviceBuffer(4096)

    def read_ceiling(names, per):
        def launches():
            for l in range(args.rotate):
                mimg.stream_read_dev([(layers[l][name].info()[0], weight_bytes(*next((c[1], c[2], c[3])
                                                                               for c in CFG1 if c[0] == name)))
                                      for name in names], per, sink.ptr, stream.handle)

        g = hiprt.Graph(stream, launches)
        for _ in range(2):
            g.launch(stream)
        a, b = hiprt.Event(), hiprt.Event()
        a.record(stream)
        for _ in range(args.roofline_replays):
            g.launch(stream)
        b.record(stream)
        b.sync()
        g.destroy()
        return a.elapsed_ms(b) * 1e3 / (args.roofline_replays * args.rotate)

    gu_weight_bytes = sum(weight_bytes(c[1], c[2], c[3]) for c in CFG1 if c[0] in ("gate", "up"))
    ceil = {per: read_ceiling(["gate", "up"], per) for per in (4, 8, 16)}
    c_per = min(ceil, key=ceil.get)
    c_us = ceil[c_per]
    c_gbs = gu_weight_bytes / (c_us * 1e-6) / 1e9
    log(f"  read ceiling (gate+up weight bytes, one launch): {c_us:.2f} us, {c_gbs:.0f} GB/s "
        f"({', '.join(f'{p}x16B: {u:.2f} us' for p, u in ceil.items())})")
    set_weight_bytes = sum(weight_bytes(c[1], c[2], c[3]) for c in CFG1)
    if use_set_roof:
        sceil = {per: read_ceiling([c[0] for c in CFG1], per) for per in (4, 8, 16)}
        sc_per = min(sceil, key=sceil.get)
        sc_us = sceil[sc_per]
        sc_gbs = set_weight_bytes / (sc_us * 1e-6) / 1e9
        log(f"  read ceiling (the seven matrices' weight bytes, one launch): {sc_us:.2f} us, {sc_gbs:.0f} GB/s")

    # An HBM ceiling independent of this library's read kernel, in the same
    # run: a 1 GiB device-to-device hipMemcpyAsync (the runtime's own copy;
    # it reads and writes 1 GiB), beside the read kernel over the same 1 GiB
    # (one launch, so its ramp and drain weigh less than at 66 MB).
    big = 1 << 30
    src_big, dst_big = hiprt.DeviceBuffer(big), hiprt.DeviceBuffer(big)
    hiprt.check(hiprt.rt().hipMemsetAsync(ctypes.c_void_p(src_big.ptr), 1, big, ctypes.c_void_p(stream.handle)), "memset")

    def timed_us(fn, reps=5):
        fn()
        a, b = hiprt.Event(), hiprt.Event()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        b.sync()
        return a.elapsed_ms(b) * 1e3 / reps

    copy_us = timed_us(lambda: hiprt.check(hiprt.rt().hipMemcpyAsync(
        ctypes.c_void_p(dst_big.ptr), ctypes.c_void_p(src_big.ptr), big, hiprt.D2D, ctypes.c_void_p(stream.handle)),
        "hipMemcpyAsync"))
    read_big_us = {per: timed_us(lambda: mimg.stream_read_dev([(src_big.ptr, big)], per, sink.ptr, stream.handle))
                   for per in (4, 8, 16)}
    rb_per = min(read_big_us, key=read_big_us.get)
    src_big.free()
    dst_big.free()
    hbm_ceiling = {
        "d2d_copy_1GiB": {"us": round(copy_us, 2), "GB_per_s": round(2 * big / (copy_us * 1e-6) / 1e9, 1),
                          "bytes_moved": 2 * big, "note": "hipMemcpyAsync device to device: reads and writes 1 GiB"},
        "read_kernel_1GiB": {"us": round(read_big_us[rb_per], 2), "loads_per_thread": rb_per,
                             "GB_per_s": round(big / (read_big_us[rb_per] * 1e-6) / 1e9, 1)},
    }
    log(f"  HBM ceiling: 1 GiB d2d copy {copy_us:.1f} us ({hbm_ceiling['d2d_copy_1GiB']['GB_per_s']:.0f} GB/s "
        f"read+write); read kernel over 1 GiB {read_big_us[rb_per]:.1f} us "
        f"({hbm_ceiling['read_kernel_1GiB']['GB_per_s']:.0f} GB/s)")

    # the single 4096 x 4096 Q4_K product (the q matrix,
    # weight seed 0) of one activation row (seed 1), as the reference calls
    # it: dequant_matmul_a8.v2, x quantized inside the one-row launch; a
    # graph of --rotate calls over the rotation copies.
    x0 = hiprt.DeviceBuffer.from_array(np.random.default_rng(1).standard_normal((1, 4096), dtype=np.float32))
    y0 = hiprt.DeviceBuffer(4096 * 4)

    def cfg0_launches():
        for l in range(args.rotate):
            mimg.linear_a8_group_dev([layers[l]["q"]], x0.ptr, 1, None, 256, [y0.ptr], ws[0].ptr, ws_bytes[0],
                                     stream.handle)

    g0 = hiprt.Graph(stream, cfg0_launches)
    g0.launch(stream)
    a0, b0 = hiprt.Event(), hiprt.Event()
    a0.record(stream)
    for _ in range(args.roofline_replays):
        g0.launch(stream)
    b0.record(stream)
    b0.sync()
    g0.destroy()
    cfg0_us = a0.elapsed_ms(b0) * 1e3 / (args.roofline_replays * args.rotate)
    cfg0_bytes = weight_bytes(4096, 4096, Q4_K) + 4096 * 4 + 4096 * 4
    cfg0_gbs = cfg0_bytes / (cfg0_us * 1e-6) / 1e9
    log(f"  cfg0 (Q4_K 4096x4096, M=1, a8 block 256, one call): {cfg0_us:.2f} us, {cfg0_gbs:.0f} GB/s")
    log(f"  gate+up GEMV (Q4_K 2x14336x4096, one launch): {r_us:.2f} us/launch, {r_gbs:.0f} GB/s; "
        f"gate alone: {g_us:.2f} us, {g_gbs:.0f} GB/s; down GEMV (Q6_K 4096x14336): {d_us:.2f} us/launch, "
        f"{d_gbs:.0f} GB/s")

    prefill_res, prefill_q8, prefill_f32 = run_prefills()

    # The host-memory entry point a cgo caller uses (x copied in, y copied
    # back, the call returns when y is in host memory): PCIe- and
    # synchronisation-inclusive time per gate call, for reference only.
    hx = xs[2]
    mimg.dequant_matmul_a8(layers[0]["gate"], hx)
    t0 = time.perf_counter()
    for i in range(args.rotate * 2):
        mimg.dequant_matmul_a8(layers[i % args.rotate]["gate"], hx)
    host_us = (time.perf_counter() - t0) * 1e6 / (args.rotate * 2)
    log(f"  host-memory call (gate, x and y over PCIe, synchronous): {host_us:.1f} us/call")

    # HBM bytes per launch of the same kernel at the same shape, from the
    # rocprofv3 FETCH_SIZE / WRITE_SIZE passes summarised in profiles/ (the
    # counters cannot be read from inside this process).
    def traffic_of(which):
        tpath = os.path.join(ROOT, "profiles", f"{which}_m{M}_traffic.md")
        if os.path.exists(tpath):
            for line in open(tpath):
                if line.startswith("bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
        return None

    gate_up = {"kernel": f"{'gemv_a8k_mfma_kernel<Q4_K>' if M >= 5 else f'gemv_a8k_pairs_kernel<Q4_K,M={M}>'}: "
                         "gate and up (2 x 14336x4096) in one launch as the grouped call makes them, pre-quantized "
                         "activations",
               "launch_bytes": r_bytes, "avg_launch_us": round(r_us, 3), "achieved": round(r_gbs, 1),
               "frac": round(r_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of("gemv_pairs_q4k_gateup"),
               "kernel_over_ceiling": round(r_gbs / c_gbs, 4)}
    gate_alone = {"avg_launch_us": round(g_us, 3), "launch_bytes": g_bytes, "achieved": round(g_gbs, 1),
                  "traffic": traffic_of("gemv_pairs_q4k_gate")}
    q6k_down = {"avg_launch_us": round(d_us, 3), "launch_bytes": d_bytes, "achieved": round(d_gbs, 1)}
    gu_ceiling = {"kernel": "stream_read_kernel (mimg_stream_read_dev): the gate and up weight bytes read in one "
                            "launch, 16-byte nontemporal loads, nothing computed",
                  "bytes": gu_weight_bytes, "avg_launch_us": round(c_us, 3), "achieved": round(c_gbs, 1),
                  "frac": round(c_gbs / HBM_PEAK_GBS, 4), "loads_per_thread": c_per}
    if use_set_roof:
        roofline = {
            "bound": "hbm", "achieved": round(s_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(s_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of("gemv_set_cfg1"),
            "kernel": "gemv_a8k_set_kernel: the seven cfg1 products (Q4_K and Q6_K) in one launch as the set "
                      "step runs them, rows quantized beforehand",
            "launch_bytes": s_bytes, "avg_launch_us": round(s_us, 3),
            "read_ceiling": {"kernel": "stream_read_kernel (mimg_stream_read_dev): the seven matrices' weight bytes "
                                       "read in one launch, 16-byte nontemporal loads, nothing computed",
                             "bytes": set_weight_bytes, "avg_launch_us": round(sc_us, 3),
                             "achieved": round(sc_gbs, 1), "frac": round(sc_gbs / HBM_PEAK_GBS, 4),
                             "loads_per_thread": sc_per, "kernel_over_ceiling": round(s_gbs / sc_gbs, 4)},
            "gate_up": gate_up, "gate_alone": gate_alone, "q6k_down": q6k_down, "gate_up_read_ceiling": gu_ceiling,
            "hbm_ceiling": hbm_ceiling,
        }
    else:
        roofline = {
            "bound": "hbm", "achieved": round(r_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r_gbs / HBM_PEAK_GBS, 4), "traffic": gate_up["traffic"], "kernel": gate_up["kernel"],
            "launch_bytes": r_bytes, "avg_launch_us": round(r_us, 3), "gate_alone": gate_alone,
            "q6k_down": q6k_down, "read_ceiling": dict(gu_ceiling, kernel_over_ceiling=gate_up["kernel_over_ceiling"]),
            "hbm_ceiling": hbm_ceiling,
        }
    step_forms = {"set": "the four groups' rows quantized in one launch, the seven products in one launch "
                         "(mimg_linear_a8_set_dev; the inputs are independent)",
                  "group": "one launch per grouped call (q/k/v, o, gate/up, down), as a decoder layer calls them",
                  "chain": "the four grouped calls as one chain launch"}
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x q4_k/q6_k, i32 block sums, f32 epilogue",
        "data": "synthetic (W ~ N(0,0.02^2) seeds 0..6 encoded Q4_K/Q6_K; x ~ N(0,1) seeds 100..103)",
        "config": {
            "workload": f"cfg1: Llama-3-8B decoder-layer linear set, M={M}, Q4_K_M (q,k,o,gate,up Q4_K; v,down Q6_K), "
                        "dequant_matmul_a8.v2 block=256",
            "rows": M,
            "step": step_kind,
            "step_form": step_forms[step_kind],
            "bytes_per_step": step_bytes(M),
            "rotation_layers": args.rotate,
            "graphs": not args.eager,
            "steps_per_graph": gs,
            "other_forms_us_per_step": other_us,
            "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
        "cfg0": {
            "workload": "cfg0: one 4096x4096 Q4_K product (weight seed 0) of one activation row (seed 1), "
                        "dequant_matmul_a8.v2 block 256, quantized inside the launch",
            "bytes": cfg0_bytes,
            "us_per_call": round(cfg0_us, 3),
            "GB_per_s": round(cfg0_gbs, 1),
            "hbm_fraction": round(cfg0_gbs / HBM_PEAK_GBS, 4),
        },
        "prefill": {
            "workload": "cfg2: gate 14336x4096 Q4_K and down 4096x14336 Q6_K, dequant_matmul_a8.v2 block=256, "
                        "int8 MFMA GEMM (bit-identical to the GEMV), activations quantized beforehand",
            "results": prefill_res,
        },
        "prefill_q8_0": {
            "workload": "cfg2's Q8_0 variant: gate 14336x4096 and down 4096x14336 Q8_0 (62 MB each), "
                        "dequant_matmul_a8.v1 (activation blocks of 32) on the int8 MFMA GEMM "
                        "(mimg_matmul_a8_quantized_q8_0_tiled_dev, opt-in: one float chain of exact block sums, "
                        "within the spec's a8 tolerance), activations quantized beforehand",
            "results": prefill_q8,
        },
        "prefill_kquant_b32": {
            "workload": "cfg2's gate (Q4_K) and down (Q6_K) with activation blocks of 32 (a dequant_matmul_a8.v1 "
                        "graph) on the int8 MFMA GEMM (mimg_matmul_a8_quantized_b32_tiled_dev, opt-in: the "
                        "reference's per-block form with one float chain, within the spec's a8 tolerance), "
                        "activations quantized beforehand",
            "results": prefill_b32,
        },
        "prefill_f32": {
            "workload": "the same gate/down products with float32 activations (dequant_matmul.v1) on the fp32 "
                        "matrix cores, within the spec bound (K+1)u sum|xw|",
            "results": prefill_f32,
        },
        "host_api": {
            "entry": "mimg_dequant_matmul_a8 (gate, host x and y)",
            "us_per_call": round(host_us, 2),
            "GB_per_s": round(launch_bytes(CFG1[4][1], CFG1[4][2], Q4_K, M) / (host_us * 1e-6) / 1e9, 1),
        },
    }
    layers.clear()
    decode_res = {}
    for name in [d for d in args.decode.split(",") if d]:
        decode_res.update(decode_bench(name, log, graph=not args.eager, cpu=not args.no_cpu,
                                       batches=[int(b) for b in args.decode_batches.split(",") if b],
                                       new_tokens=args.decode_tokens))
    if decode_res:
        result["decode"] = decode_res
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(host_bytes, xs, args.cpu_seconds, log)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
