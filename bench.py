#!/usr/bin/env python3
"""Throughput of the quantized linear-layer matmul on one MI355X.

Workload (one "step"): the linears of the Whisper large-v3 encoder at one
30 s window, M = 1500 rows, weights in Q5_1 -- 32 layers x {q, k, v, out
[1280x1280], fc1 [5120x1280], fc2 [1280x5120]}, with biases where Whisper has
them (no bias on k).  Each layer quantizes its three distinct inputs (the
attention-block input shared by q/k/v, the attention output, the MLP input)
and the fc1 output, then runs the six products in four GEMM launches (q, k
and v read one input and share a launch, as rw_rocm_matmul_prequant_multi_dev
allows).  Weights are seeded N(0, 0.02)
quantized to Q5_1 (472 MB resident, more than the 256 MB MALL); activations
are seeded N(0, 1) and resident in HBM before timing starts.

Reported: whole-step TOPS (2*M*N*K per linear), the GEMM kernel's own rate
against the MI355X f16 MFMA peak (HIP events around bursts of back-to-back
launches), the
decode-GEMV bandwidth for the large-v3 decoder linear set at M = 5 in Q5_0,
and the reference CPU path (oracle/cpu_baseline.c, AVX-512 VNNI / AVX2
restatement of matmul_t_q) timed on this host on one encoder layer.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q-matmul TOPS @M=1500 encoder; decode GEMV HBM GB/s @M=5 (large-v3 Q5_1)"
F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
HBM_PEAK_GBS = 8000.0    # MI355X HBM3E


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def encoder_workload(A, synth, torch, dtype: int, m: int, seed0: int):
    cfg = synth.LARGE_V3
    d, fc, layers = cfg["d"], cfg["fc"], cfg["layers"]
    shapes = synth.encoder_layer_shapes(d, fc)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed0)
    layers_w = []
    t0 = time.time()
    workers = min(16, os.cpu_count() or 1)
    for layer in range(layers):
        specs = [(dtype, n, k, seed0 + 100 * layer + i) for i, (_, n, k) in enumerate(shapes)]
        raws = synth.normal_weights_many(specs, workers)
        layers_w.append({name: A.DeviceWeight(dtype, n, k, raw) for (name, n, k), raw in zip(shapes, raws)})
    log(f"encoder weights uploaded ({layers} layers, {time.time() - t0:.1f} s)")
    inputs = {
        "qkv": torch.randn(m, d, device=dev, generator=g),
        "attn": torch.randn(m, d, device=dev, generator=g),
        "mlp": torch.randn(m, d, device=dev, generator=g),
        "h": torch.randn(m, fc, device=dev, generator=g),
    }
    bias = {name: (None if name == "k" else torch.randn(n, device=dev, generator=g) * 0.1)
            for name, n, _ in shapes}
    outs = {name: torch.empty(m, n, device=dev) for name, n, _ in shapes}
    wsz = {key: A.workspace_size(m, t.shape[1]) for key, t in inputs.items()}
    wsp = {key: torch.empty(wsz[key], dtype=torch.uint8, device=dev) for key in inputs}
    ops = layers * sum(2 * m * n * k for _, n, k in shapes)
    return dict(layers=layers_w, inputs=inputs, bias=bias, outs=outs, wsz=wsz, wsp=wsp, ops=ops, shapes=shapes,
                m=m, d=d, fc=fc)

SRC = {"q": "qkv", "k": "qkv", "v": "qkv", "out": "attn", "fc1": "mlp", "fc2": "h"}
# the launches of one layer: q, k and v read one input and share a launch
LAUNCHES = [("qkv", ("q", "k", "v")), ("out", ("out",)), ("fc1", ("fc1",)), ("fc2", ("fc2",))]


def product(A, W, lw, names, stream):
    m = W["m"]
    src = W["wsp"][SRC[names[0]]]
    if len(names) == 1:
        lw[names[0]].matmul_prequant_dev(src, m, W["outs"][names[0]], W["bias"][names[0]], stream)
    else:
        A.matmul_prequant_multi_dev([lw[x] for x in names], src, m, [W["outs"][x] for x in names],
                                    [W["bias"][x] for x in names], stream)


def encoder_step(A, W, stream):
    m = W["m"]
    for lw in W["layers"]:
        for key in ("qkv", "attn", "mlp", "h"):
            t = W["inputs"][key]
            A.quantize_dev(t, m, t.shape[1], W["wsp"][key], W["wsz"][key], stream)
        for _, names in LAUNCHES:
            product(A, W, lw, names, stream)


def time_encoder(A, torch, W, steps: int, warmup: int, stream):
    for _ in range(warmup):
        encoder_step(A, W, stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        encoder_step(A, W, stream)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    return ms, wall


def time_encoder_graph(A, torch, W, steps: int, warmup: int):
    """The same step captured once in a HIP graph (torch.cuda.CUDAGraph over
    the library's launches) and replayed: launches without host overhead,
    as an encoder runs window after window."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        encoder_step(A, W, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        encoder_step(A, W, torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    del graph
    return ms


def time_gemm_kernel(A, torch, W, stream, reps: int = 3):
    """Average k_gemm launch duration: per launch of the layer (q/k/v
    together, out, fc1, fc2), the launches of every layer back to back
    between two HIP events on torch's current stream (the stream the kernels
    run on), so each weight is read once per pass as in the step.  An event
    pair around every single launch would add the event packets' own latency
    to each launch; back-to-back launches on one stream leave no measurable
    gap, so the burst average is the kernel's duration.  Returns (mean launch
    ms, ops per launch, launches, per-launch mean us)."""
    m = W["m"]
    for key in ("qkv", "attn", "mlp", "h"):
        t = W["inputs"][key]
        A.quantize_dev(t, m, t.shape[1], W["wsp"][key], W["wsz"][key], stream)
    torch.cuda.synchronize()
    dims = {name: (n, k) for name, n, k in W["shapes"]}
    total_ms, ops, launches, per_launch = 0.0, 0, 0, {}
    for label, names in LAUNCHES:
        def burst():
            for lw in W["layers"]:
                product(A, W, lw, names, stream)
        burst()  # warm
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            burst()
        e1.record()
        torch.cuda.synchronize()
        cnt = reps * len(W["layers"])
        ms = e0.elapsed_time(e1)
        per_launch[label] = round(1e3 * ms / cnt, 2)
        total_ms += ms
        ops += cnt * sum(2 * m * dims[x][0] * dims[x][1] for x in names)
        launches += cnt
    return total_ms / launches, ops / launches, launches, per_launch


def decode_workload(A, synth, torch, dtype: int, m: int, seed0: int):
    cfg = synth.LARGE_V3
    d, fc, layers, vocab = cfg["d"], cfg["fc"], cfg["layers"], cfg["n_vocab"]
    shapes = synth.decoder_layer_shapes(d, fc) * layers + [("logits", vocab, d)]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed0)
    t0 = time.time()
    items, keep = [], []
    wbytes = 0
    io_bytes = 0
    workers = min(16, os.cpu_count() or 1)
    for c0 in range(0, len(shapes), 16):
        chunk = shapes[c0:c0 + 16]
        raws = synth.normal_weights_many([(dtype, n, k, seed0 + c0 + j) for j, (_, n, k) in enumerate(chunk)],
                                         workers)
        for (name, n, k), raw in zip(chunk, raws):
            items.append(_decode_item(A, torch, dev, g, dtype, name, n, k, raw, m, keep))
            wbytes += n * (k // 32) * synth.BLOCK_BYTES[dtype]
            io_bytes += 4 * m * k + 4 * m * n
    arr = A.make_linears(items)
    wsz = A.grouped_workspace_size(arr)
    ws = torch.empty(wsz, dtype=torch.uint8, device=dev)
    log(f"decoder weights uploaded ({len(shapes)} linears, {wbytes / 1e6:.1f} MB, {time.time() - t0:.1f} s)")
    return dict(arr=arr, ws=ws, wsz=wsz, keep=keep, bytes=wbytes + io_bytes, wbytes=wbytes, count=len(shapes))


def _decode_item(A, torch, dev, g, dtype, name, n, k, raw, m, keep):
    w = A.DeviceWeight(dtype, n, k, raw)
    a = torch.randn(m, k, device=dev, generator=g)
    b = None if name.endswith(".k") or name == "logits" else torch.randn(n, device=dev, generator=g) * 0.1
    o = torch.empty(m, n, device=dev)
    keep += [w, a, b, o]
    return (w, a, b, o, m)


def time_decode(A, torch, D, steps: int, warmup: int, stream):
    """ms per pass over the whole decoder linear set: (prepared group, one
    grouped call that also uploads its launch tables)."""
    group = A.Group(D["arr"])

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    t_group = timed(lambda: group.run(stream))
    t_call = timed(lambda: A.matmul_grouped_dev(D["arr"], D["ws"], D["wsz"], stream))
    group.free()
    return t_group, t_call


def time_attention(A, torch, stream, steps: int, warmup: int, t: int = 1500, n_state: int = 1280, n_head: int = 20):
    """One encoder layer's self-attention (large-v3: 20 heads of 64 over 1500
    positions) through rw_rocm_attention_dev on resident q, k, v: ms per
    call (the three split launches and k_attn) and the algorithmic flops
    (2 t^2 dh per head for Q K^T, the same for P V)."""
    g = torch.Generator(device="cuda:0")
    g.manual_seed(11)
    q, k, v = (torch.randn(t, n_state, device="cuda:0", generator=g) for _ in range(3))
    out = torch.empty(t, n_state, device="cuda:0")
    wsz = A.attention_workspace_size(t, t, n_state)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")

    def call():
        A.attention_dev(q, k, v, t, t, n_state, n_head, False, out, workspace=ws, workspace_len=wsz, stream=stream)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 4 * t * t * (n_state // n_head) * n_head
    return ms, flops


def time_encoder_layers(A, torch, W, stream, steps: int, warmup: int):
    """All 32 large-v3 encoder layers end to end on the device
    (rw_rocm_encoder_layer_dev per layer: layernorms, the four products,
    attention, GELU and the residual adds) on one resident [1500, 1280]
    activation; the weights are the workload's, the layernorm and bias
    vectors random.  Returns ms per pass over all layers."""
    m, d, fc = W["m"], W["d"], W["fc"]
    g = torch.Generator(device="cuda:0")
    g.manual_seed(21)
    vec = lambda k, c: (torch.randn(k, device="cuda:0", generator=g) * 0.1 + c)  # noqa: E731
    layers = []
    for lw in W["layers"]:
        layers.append(A.EncoderLayer(d // 64, q=lw["q"], k=lw["k"], v=lw["v"], out=lw["out"], fc1=lw["fc1"],
                                     fc2=lw["fc2"], attn_ln_w=vec(d, 1.0), attn_ln_b=vec(d, 0.0),
                                     q_b=W["bias"]["q"], v_b=W["bias"]["v"], out_b=W["bias"]["out"],
                                     mlp_ln_w=vec(d, 1.0), mlp_ln_b=vec(d, 0.0), fc1_b=W["bias"]["fc1"],
                                     fc2_b=W["bias"]["fc2"]))
    x0 = torch.randn(m, d, device="cuda:0", generator=g)
    x = x0.clone()
    wsz = layers[0].workspace_size(m)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")

    def run(s):
        x.copy_(x0)
        for L in layers:
            L.run(x, m, ws, wsz, s)

    def timed(fn):
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    for _ in range(warmup):
        run(stream)
    eager = timed(lambda: run(stream))
    ok = bool(torch.isfinite(x).all().item())
    ref = x.clone()
    # the same pass captured once and replayed (every launch is a kernel: no
    # memset, no host wait), checked against the eager result
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        run(cs.cuda_stream)  # warm the capture stream's allocations
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=cs):
            run(cs.cuda_stream)
    torch.cuda.current_stream().wait_stream(cs)
    graph = timed(g.replay)
    ok = ok and bool(torch.equal(x, ref))
    return eager, graph, ok


def time_decoder_tokens(A, synth, torch, D, stream, steps: int):
    """The large-v3 decoder on the device, one beam: rw_decoder with the
    decode workload's weights (32 layers x 10 linears, the token embedding as
    both embedding and logits head), random layernorm and bias vectors, a
    [1500, 1280] encoder output.  Returns (ms for set_audio, ms per token
    for forward_hidden + the logits product)."""
    cfg = synth.LARGE_V3
    d, layers, vocab = cfg["d"], cfg["layers"], cfg["n_vocab"]
    keep = D["keep"]
    per = 10  # linears per layer, in decoder_layer_shapes order
    names = ("q", "k", "v", "out", "cq", "ck", "cv", "cout", "fc1", "fc2")
    g = torch.Generator(device="cuda:0")
    g.manual_seed(31)
    vec = lambda k, c=0.0: torch.randn(k, device="cuda:0", generator=g) * 0.1 + c  # noqa: E731
    lay = []
    for l in range(layers):
        L = {nm: keep[4 * (per * l + i)] for i, nm in enumerate(names)}
        for nm in ("attn_ln", "cross_ln", "mlp_ln"):
            L[nm + "_w"], L[nm + "_b"] = vec(d, 1.0), vec(d)
        for nm in ("q_b", "v_b", "out_b", "cq_b", "cv_b", "cout_b", "fc2_b"):
            L[nm] = vec(d)
        L["fc1_b"] = vec(4 * d)
        lay.append(L)
    emb = keep[4 * per * layers]
    dec = A.Decoder(d // 64, 448, 1500, lay, emb, vec(448 * d), vec(d, 1.0), vec(d))
    enc = torch.randn(1500, d, device="cuda:0", generator=g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.set_audio(enc, stream)
    torch.cuda.synchronize()
    t_audio = (time.perf_counter() - t0) * 1e3
    hid = torch.empty(4, d, device="cuda:0")
    logits = torch.empty(1, vocab, device="cuda:0")
    dec.forward_hidden([50258, 50259, 50359], hid[:3], stream)
    tok = 50363

    def one():
        dec.forward_hidden([tok], hid[:1], stream)
        emb.matmul_dev(hid[:1], 1, logits, stream=stream)

    one()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        one()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ok = bool(torch.isfinite(logits).all().item())
    dec.free()
    return t_audio, ms, ok


def time_model_load(A, synth, dtype: int, path: str, reps: int = 2):
    """rw_rocm_model_load on a ggml .bin holding large-v3's quantized matrices
    (32 encoder layers x 6 linears, 32 decoder layers x 10, the token
    embedding [51866, 1280]) as random blocks: parse the map, upload and
    repack every matrix.  The file is freshly written, so it is read from the
    page cache; returns (seconds per load, file bytes, matrices)."""
    import struct

    import numpy as np

    cfg = synth.LARGE_V3
    d, fc, layers = cfg["d"], cfg["fc"], cfg["layers"]
    shapes = [(f"encoder.blocks.{i}.{nm}.weight", n, k) for i in range(layers)
              for nm, n, k in synth.encoder_layer_shapes(d, fc)]
    shapes += [(f"decoder.blocks.{i}.{nm}.weight", n, k) for i in range(layers)
               for nm, n, k in synth.decoder_layer_shapes(d, fc)]
    shapes.append(("decoder.token_embedding.weight", cfg["n_vocab"], d))
    rng = np.random.default_rng(7)
    bb = synth.BLOCK_BYTES[dtype]
    i32 = lambda v: struct.pack("<i", v)  # noqa: E731
    with open(path, "wb") as f:
        hp = [cfg["n_vocab"], 1500, d, 20, layers, 448, d, 20, layers, 128, 1]
        f.write(i32(0x67676D6C) + b"".join(i32(v) for v in hp) + i32(0) + i32(0) + i32(0))
        for name, n, k in shapes:
            nm = name.encode()
            f.write(i32(2) + i32(len(nm)) + i32(dtype) + i32(k) + i32(n) + nm)
            blocks = rng.integers(0, 256, size=(n * k // 32, bb), dtype=np.uint8)
            blocks[:, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)  # finite scales
            f.write(blocks.tobytes())
        size = f.tell()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        M = A.Model(path)
        times.append(time.perf_counter() - t0)
        M.free()
    os.unlink(path)
    return min(times), size, len(shapes)


def cpu_baseline(synth, dtype: int, m: int, budget_s: float):
    """The reference CPU path (oracle/cpu_baseline.c) on one large-v3 encoder
    layer: each of the six linears on its first call (cold path, as the
    encoder runs in production), median of repeated runs."""
    import numpy as np

    import oracle as O

    cfg = synth.LARGE_V3
    shapes = synth.encoder_layer_shapes(cfg["d"], cfg["fc"])
    threads = O.cpu_threads()
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit():
        threads = min(threads, int(cap))
    rng = np.random.default_rng(7)
    raws = [synth.normal_weights(dtype, n, k, seed=900 + i) for i, (_, n, k) in enumerate(shapes)]
    acts = {k: rng.standard_normal((m, k)).astype(np.float32) for k in {k for _, _, k in shapes}}
    per_linear = [[] for _ in shapes]
    t_start = time.time()
    reps = 0
    while reps < 5 and (reps < 1 or time.time() - t_start < budget_s):
        for i, (_, n, k) in enumerate(shapes):
            t = O.CpuQTensor(dtype, n, k, raws[i])
            t0 = time.perf_counter()
            t.matmul(acts[k], threads=threads)
            per_linear[i].append(time.perf_counter() - t0)
            tier = t.tier_used
            t.close()
        reps += 1
    layer_s = sum(statistics.median(v) for v in per_linear)
    ops = sum(2 * m * n * k for _, n, k in shapes)
    tier_name = {0: "avx512-vnni", 1: "avx2", 2: "f32"}[tier]
    return {
        "value": round(ops / layer_s / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"one large-v3 encoder layer (6 Q5_1 linears, M={m}), cold path, median of {reps} runs "
                  f"per linear, tier {tier_name}, {threads} threads",
        "layer_ms": round(layer_s * 1e3, 2),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--m", type=int, default=1500)
    ap.add_argument("--quant", default="Q5_1")
    ap.add_argument("--decode-quant", default="Q5_0")
    ap.add_argument("--decode-m", type=int, default=5)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--no-layers", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--load-model", default="",
                    help="also time the model loader on a large-v3-shaped ggml file written to this path")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="first copy this many MiB device to device (a kernel of known traffic, to scale "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the library has no multi-GPU path.",
              file=sys.stderr)
        return 2

    import torch

    from rusty_whisper_amd import _abi as A
    from rusty_whisper_amd import synth

    A.init(0)
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream().cuda_stream
    if args.copy_probe_mb:
        src = torch.ones(args.copy_probe_mb << 18, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe_mb} MiB read + {args.copy_probe_mb} MiB written")
        del src, dst
    dtype = synth.BY_NAME[args.quant]

    W = encoder_workload(A, synth, torch, dtype, args.m, seed0=1)
    eager_ms, wall = time_encoder(A, torch, W, args.steps, args.warmup, stream)
    eager_tops = W["ops"] / (eager_ms * 1e-3) / 1e12
    log(f"encoder step, eager launches {eager_ms:.3f} ms  ({eager_tops:.1f} TOPS, wall {wall:.2f} s)")
    ms = time_encoder_graph(A, torch, W, args.steps, args.warmup)
    tops = W["ops"] / (ms * 1e-3) / 1e12
    log(f"encoder step, graph replay {ms:.3f} ms  ({tops:.1f} TOPS)")

    gemm_ms, gemm_ops, launches, per_shape = time_gemm_kernel(A, torch, W, stream)
    gemm_tops = gemm_ops / (gemm_ms * 1e-3) / 1e12
    log(f"k_gemm average launch {gemm_ms * 1e3:.1f} us over {launches} launches -> {gemm_tops:.1f} TOPS "
        f"(per launch, us: {per_shape})")

    result = {
        "metric": METRIC,
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "eager_ms_per_step": round(eager_ms, 4),
        "launch": "one encoder step (256 launches: per layer 4 quantizations, q/k/v in one GEMM launch, out, "
                  "fc1, fc2) captured in a HIP graph and replayed; eager_ms_per_step launches the same kernels "
                  "one by one from the host",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"large-v3 encoder linears, {args.quant}, M={args.m}: 32 layers x "
                        f"(q,k,v,out 1280x1280; fc1 5120x1280; fc2 1280x5120), activations quantized on device "
                        f"to int8 blocks as the reference does, products on f16 MFMA (dequantized operands, "
                        f"f32 accumulation)",
            "m": args.m,
            "layers": 32,
            "quant": args.quant,
            "ops_per_step": W["ops"],
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(gemm_tops, 3),
            "peak": F16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tops / F16_PEAK_TFLOPS, 4),
            "traffic": None,
            "kernel": f"k_gemm<{args.quant}> on v_mfma_f32_32x32x16_f16 (2*M*N*K per launch)",
            "avg_launch_us": round(gemm_ms * 1e3, 2),
            "launch_us_by_launch": per_shape,
            "frac_of_int8_peak": round(gemm_tops / INT8_PEAK_TOPS, 4),
        },
    }
    if not args.no_layers:
        eager_l, lms, finite = time_encoder_layers(A, torch, W, stream, max(3, args.steps // 2), 1)
        log(f"32 encoder layers on the device: graph replay {lms:.3f} ms ({lms * 1e3 / 32:.1f} us per layer), "
            f"eager {eager_l:.3f} ms (finite and replay == eager: {finite})")
        result["encoder_layers"] = {
            "workload": f"large-v3 encoder, 32 layers, {args.quant}, M={args.m}: per layer layernorm + q/k/v + "
                        "attention (20 heads) + out + residual, layernorm + fc1 + GELU + fc2 + residual, all on the "
                        "device (rw_rocm_encoder_layer_dev), captured in a HIP graph and replayed",
            "ms_per_pass": round(lms, 4),
            "us_per_layer": round(lms * 1e3 / 32, 2),
            "eager_ms_per_pass": round(eager_l, 4),
            "finite_and_replay_equal": finite,
        }

    del W
    torch.cuda.empty_cache()

    if not args.no_decode:
        D = decode_workload(A, synth, torch, synth.BY_NAME[args.decode_quant], args.decode_m, seed0=5000)
        dms, dms_call = time_decode(A, torch, D, max(3, args.steps), 2, stream)
        gbs = D["bytes"] / (dms * 1e-3) / 1e9
        log(f"decode set {dms:.3f} ms ({gbs:.1f} GB/s); with per-call table upload {dms_call:.3f} ms")
        result["decode"] = {
            "metric": f"decode GEMV HBM GB/s @M={args.decode_m}",
            "workload": f"large-v3 decoder linears, {args.decode_quant}, M={args.decode_m}: 32 layers x 10 "
                        f"linears + logits [51866x1280], {D['count']} independent linears per step",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(dms, 4),
            "ms_per_step_with_table_upload": round(dms_call, 4),
            "bytes_per_step": D["bytes"],
            "launch": "prepared group (rw_rocm_group_run): one k_gemv_records launch (each linear's activation quantized once) and one k_gemv launch for the set",
            "peak": HBM_PEAK_GBS,
            "frac": round(gbs / HBM_PEAK_GBS, 4),
        }
        if not args.no_layers:
            t_audio, tok_ms, finite = time_decoder_tokens(A, synth, torch, D, stream, 20)
            log(f"decoder on the device: set_audio {t_audio:.2f} ms, {tok_ms:.3f} ms per token with logits "
                f"(finite={finite})")
            result["decoder_tokens"] = {
                "workload": "large-v3 decoder, one beam, Q5_0: per token the embedding, 32 layers (causal "
                            "self-attention over the cache, cross-attention to 1500 positions, MLP), final "
                            "layernorm and the [51866 x 1280] logits product, all on the device (rw_decoder)",
                "ms_per_token": round(tok_ms, 4),
                "set_audio_ms": round(t_audio, 3),
                "finite": finite,
            }
        del D
        torch.cuda.empty_cache()

    if not args.no_attention:
        ams, aflops = time_attention(A, torch, stream, max(5, args.steps), 2)
        atf = aflops / (ams * 1e-3) / 1e12
        log(f"encoder self-attention {ams * 1e3:.1f} us per layer ({atf:.1f} TFLOP/s algorithmic)")
        result["attention"] = {
            "workload": "large-v3 encoder self-attention, one layer: 20 heads x 64, 1500 positions, f32 in/out",
            "us_per_layer": round(ams * 1e3, 2),
            "flops": aflops,
            "TFLOP_per_s": round(atf, 2),
            "launch": "rw_rocm_attention_dev: one split launch (q, k, v to f16 hi/lo planes) and one k_attn",
            "note": "algorithmic flops 4*t^2*64 per head; each product runs as three f16 MFMA products",
        }

    if args.load_model:
        lq = synth.BY_NAME[args.decode_quant]
        secs, size, count = time_model_load(A, synth, lq, args.load_model)
        log(f"model load {secs:.3f} s for {size / 1e9:.3f} GB ({size / secs / 1e9:.2f} GB/s, {count} matrices)")
        result["model_load"] = {
            "workload": f"ggml .bin of large-v3's {count} quantized matrices ({args.decode_quant}, random blocks), "
                        f"in the page cache: parse, upload and repack every matrix",
            "seconds": round(secs, 4),
            "file_bytes": size,
            "GB_per_s": round(size / secs / 1e9, 3),
        }

    if not args.no_cpu:
        cb = cpu_baseline(synth, dtype, args.m, args.cpu_seconds)
        log(f"cpu baseline {cb['value']} TOPS ({cb['sample']})")
        result["cpu_baseline"] = cb

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
