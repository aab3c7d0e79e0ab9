#!/usr/bin/env python3
"""Throughput of the quantized linear-layer matmul on one MI355X.

Headline workload (one "step"): the linears of the Whisper large-v3 encoder
at one 30 s window, M = 1500 rows, weights in Q5_1 -- 32 layers x {q, k, v,
out [1280x1280], fc1 [5120x1280], fc2 [1280x5120]}, with biases where
Whisper has them (no bias on k).  Each layer quantizes its three distinct
inputs (the attention-block input shared by q/k/v, the attention output, the
MLP input) and fc2's input, then runs the six products in four GEMM
launches (q, k and v read one input and share a launch, as
rw_rocm_matmul_prequant_multi_dev allows).  `fused_mlp` times the same step
with fc2's input gelu(fc1's output), as the encoder's MLP runs, quantized in
fc1's epilogue (rw_rocm_matmul_prequant_gelu_quantize_dev).  Weights are seeded N(0, 0.02)
quantized to Q5_1 (472 MB resident, more than the 256 MB MALL); activations
are seeded N(0, 1) and resident in HBM before timing starts.  `value` is the
step with the same activation buffers for every layer (warm); `cold` gives
each layer its own inputs, outputs and workspaces (2.6 GB touched per step,
ten times the MALL).

Reported beside it: the GEMM kernel's own rate against the MI355X f16 MFMA
peak (HIP events around bursts of back-to-back launches) with its HBM
traffic from the committed rocprofv3 counter summary, one leg per benchmark
configuration (tiny.en fc1; small.en Q8_0 with outliers; large-v3 Q4_0 and
Q4_1 with scale spread; the large-v3 decoder set at M = 5 and M = 1; the
turbo batch at M = 12000 and M = 40), the device encoder layers, attention
and decoder steps, and the reference CPU path (oracle/cpu_baseline.c,
AVX-512 VNNI / AVX2 restatement of matmul_t_q) timed on this host on one
encoder layer (cold path) and on decoder shapes (packed cache).
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


def encoder_workload(A, synth, torch, dtype: int, m: int, seed0: int, cfg=None, spread: bool = False,
                     outliers: float = 0.0, layers_w=None, cold: bool = False):
    """Weights (seeded N(0, 0.02), each 32-block scaled by 10**U(-1, 1) with
    `spread`), per-launch inputs (N(0, 1), `outliers` of the channels x20),
    biases, outputs and quantization workspaces for cfg's encoder linears.
    `layers_w` reuses uploaded weights of the same shapes and dtype; `cold`
    gives every layer its own inputs, outputs and workspaces."""
    cfg = cfg or synth.LARGE_V3
    d, fc, layers = cfg["d"], cfg["fc"], cfg["layers"]
    shapes = synth.encoder_layer_shapes(d, fc)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed0)
    if layers_w is None:
        layers_w = []
        t0 = time.time()
        workers = min(16, os.cpu_count() or 1)
        for layer in range(layers):
            specs = [(dtype, n, k, seed0 + 100 * layer + i, 0.02, spread) for i, (_, n, k) in enumerate(shapes)]
            raws = synth.normal_weights_many(specs, workers)
            layers_w.append({name: A.DeviceWeight(dtype, n, k, raw) for (name, n, k), raw in zip(shapes, raws)})
        log(f"encoder weights uploaded ({layers} layers of {synth.NAMES[dtype]}, d={d}, {time.time() - t0:.1f} s)")
    widths = {"qkv": d, "attn": d, "mlp": d, "h": fc}
    ch = {}
    if outliers > 0:
        for key, k in widths.items():
            idx = torch.randperm(k, generator=g, device=dev)[:max(1, int(round(outliers * k)))]
            ch[key] = idx

    def make_inputs():
        t = {key: torch.randn(m, k, device=dev, generator=g) for key, k in widths.items()}
        for key, idx in ch.items():
            t[key][:, idx] *= 20.0
        return t

    wsz = {key: A.workspace_size(m, k) for key, k in widths.items()}
    # fc2's input workspace also takes the fused GELU + quantization's quants
    wsz["h"] = max(wsz["h"], A.gelu_quantize_workspace_size(m, fc))

    def make_set():
        return dict(inputs=make_inputs(), wsp={key: torch.empty(wsz[key], dtype=torch.uint8, device=dev)
                                               for key in widths},
                    outs={name: torch.empty(m, n, device=dev) for name, n, _ in shapes})

    bias = {name: (None if name == "k" else torch.randn(n, device=dev, generator=g) * 0.1)
            for name, n, _ in shapes}
    sets = [make_set() for _ in range(layers if cold else 1)]
    ops = layers * sum(2 * m * n * k for _, n, k in shapes)
    return dict(layers=layers_w, sets=sets, bias=bias, wsz=wsz, ops=ops, shapes=shapes, m=m, d=d, fc=fc,
                inputs=sets[0]["inputs"], wsp=sets[0]["wsp"], outs=sets[0]["outs"])


SRC = {"q": "qkv", "k": "qkv", "v": "qkv", "out": "attn", "fc1": "mlp", "fc2": "h"}
# the launches of one layer: q, k and v read one input and share a launch
LAUNCHES = [("qkv", ("q", "k", "v")), ("out", ("out",)), ("fc1", ("fc1",)), ("fc2", ("fc2",))]


def product(A, W, lw, names, stream, bufs=None):
    bufs = bufs or W["sets"][0]
    m = W["m"]
    src = bufs["wsp"][SRC[names[0]]]
    if len(names) == 1:
        lw[names[0]].matmul_prequant_dev(src, m, bufs["outs"][names[0]], W["bias"][names[0]], stream)
    else:
        A.matmul_prequant_multi_dev([lw[x] for x in names], src, m, [bufs["outs"][x] for x in names],
                                    [W["bias"][x] for x in names], stream)


def encoder_step(A, W, stream, fused: bool = False):
    """One step: per layer the q/k/v input, the attention output and the MLP
    input are quantized (synthetic activations), then q/k/v (one launch), out,
    fc1 and fc2.  fused: as the encoder runs its MLP (src/encoder.rs:161-171),
    fc2's input is gelu(fc1's output), quantized in fc1's epilogue
    (rw_rocm_matmul_prequant_gelu_quantize_dev); otherwise fc1 writes its f32
    output and fc2 reads a fourth synthetic activation, quantized by its own
    launch (every product as a separate matmul_t_q call)."""
    m, sets = W["m"], W["sets"]
    keys = ("qkv", "attn", "mlp") if fused else ("qkv", "attn", "mlp", "h")
    for i, lw in enumerate(W["layers"]):
        bufs = sets[i % len(sets)]
        for key in keys:
            t = bufs["inputs"][key]
            A.quantize_dev(t, m, t.shape[1], bufs["wsp"][key], W["wsz"][key], stream)
        for label, names in LAUNCHES:
            if fused and label == "fc1":
                A.matmul_prequant_gelu_quantize_dev(lw["fc1"], bufs["wsp"]["mlp"], m, W["bias"]["fc1"],
                                                    bufs["wsp"]["h"], W["wsz"]["h"], stream)
            else:
                product(A, W, lw, names, stream, bufs)


def time_encoder(A, torch, W, steps: int, warmup: int, stream, fused: bool = False):
    for _ in range(warmup):
        encoder_step(A, W, stream, fused)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        encoder_step(A, W, stream, fused)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    return ms, wall


def time_graph(torch, fn, steps: int, warmup: int):
    """fn(stream) captured once in a HIP graph (torch.cuda.CUDAGraph over the
    library's launches) and replayed: launches without host overhead, as an
    encoder runs window after window.  Returns ms per replay."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(torch.cuda.current_stream().cuda_stream)
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


def time_encoder_graph(A, torch, W, steps: int, warmup: int, fused: bool = False):
    return time_graph(torch, lambda st: encoder_step(A, W, st, fused), steps, warmup)


def time_gemm_kernel(A, torch, W, stream, reps: int = 3):
    """Average k_gemm launch duration: per launch type of the layer (q/k/v
    together, out, fc1, fc2), the launches of every layer back to back,
    captured in one HIP graph and replayed `reps` times between two HIP
    events, so each weight is read once per pass as in the step and no host
    launch overhead sits between them (an 11 us launch is shorter than a
    launch from Python).  Back-to-back launches on one stream leave no
    measurable gap, so the burst average is the kernel's duration.  Returns
    (mean launch ms, ops per launch, launches, per-launch mean us)."""
    m = W["m"]
    for key in ("qkv", "attn", "mlp", "h"):
        t = W["inputs"][key]
        A.quantize_dev(t, m, t.shape[1], W["wsp"][key], W["wsz"][key], stream)
    torch.cuda.synchronize()
    dims = {name: (n, k) for name, n, k in W["shapes"]}
    total_ms, ops, launches, per_launch = 0.0, 0, 0, {}
    for label, names in LAUNCHES:
        def burst(st, names=names):
            for lw in W["layers"]:
                product(A, W, lw, names, st)
        ms = time_graph(torch, burst, reps, 1) * reps
        cnt = reps * len(W["layers"])
        per_launch[label] = round(1e3 * ms / cnt, 2)
        total_ms += ms
        ops += cnt * sum(2 * m * dims[x][0] * dims[x][1] for x in names)
        launches += cnt
    return total_ms / launches, ops / launches, launches, per_launch


def decode_workload(A, synth, torch, dtype: int, m: int, seed0: int, cfg=None):
    """cfg's decoder linears (10 per layer) plus the [n_vocab x d] logits,
    each with its own m-row input, output and bias (none on the k
    projections and the logits)."""
    cfg = cfg or synth.LARGE_V3
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
    log(f"decoder weights uploaded ({len(shapes)} linears, {wbytes / 1e6:.1f} MB, {time.time() - t0:.1f} s)")
    return decode_rows(A, torch, dict(items=items, keep=keep, wbytes=wbytes, count=len(shapes), m=m), m)


def _decode_item(A, torch, dev, g, dtype, name, n, k, raw, m, keep):
    w = A.DeviceWeight(dtype, n, k, raw)
    a = torch.randn(m, k, device=dev, generator=g)
    b = None if name.endswith(".k") or name == "logits" else torch.randn(n, device=dev, generator=g) * 0.1
    o = torch.empty(m, n, device=dev)
    keep += [w, a, b, o]
    return (w, a, b, o, m)


def decode_rows(A, torch, D, m: int):
    """The workload's linears on the first m of their rows (m <= D's own)."""
    items = [(w, a[:m], b, o[:m], m) for (w, a, b, o, _) in D["items"]]
    arr = A.make_linears(items)
    wsz = A.grouped_workspace_size(arr)
    io = sum(4 * m * (w.k + w.n) for (w, _, _, _, _) in D["items"])
    return dict(D, arr=arr, ws=torch.empty(wsz, dtype=torch.uint8, device="cuda:0"), wsz=wsz, rows=m,
                bytes=D["wbytes"] + io, row_items=items)


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
    n_ctx = 448
    dec = A.Decoder(d // 64, n_ctx, 1500, lay, emb, vec(n_ctx * d), vec(d, 1.0), vec(d))
    enc = torch.randn(1500, d, device="cuda:0", generator=g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.set_audio(enc, stream)
    torch.cuda.synchronize()
    t_audio_cold = (time.perf_counter() - t0) * 1e3  # host clock, first call (workspace allocation included)
    warm = []
    for _ in range(7):  # later windows: HIP events on the launching stream, median
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        dec.set_audio(enc, stream)
        e1.record()
        torch.cuda.synchronize()
        warm.append(e0.elapsed_time(e1))
    t_audio = {"cold_ms": t_audio_cold, "warm_ms": statistics.median(warm)}
    hid = torch.empty(n_ctx, d, device="cuda:0")
    logits = torch.empty(1, vocab, device="cuda:0")
    tok = 50363

    def one():
        dec.forward_hidden([tok], hid[:1], stream)
        emb.matmul_dev(hid[:1], 1, logits, stream=stream)

    # per token at three cache lengths: the steps end at n_past = `end`
    per_len = {}
    for end, timed in ((24, steps), (224, 4), (440, 4)):
        dec.reset()
        prompt = [50258, 50259, 50359] + [(440 + 37 * i) % 50000 for i in range(end - timed - 4)]
        dec.forward_hidden(prompt, hid[:len(prompt)], stream)
        one()  # warm
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(timed):
            one()
        e1.record()
        torch.cuda.synchronize()
        assert dec.n_past == end
        per_len[end] = e0.elapsed_time(e1) / timed
    ok = bool(torch.isfinite(logits).all().item())
    # beam search: 5 forks at one cache length step together
    # (rw_rocm_decoder_forward_beams_dev), then the stacked logits [5 x 51866]
    # and their log_softmax + top-5 on the device
    nb, k = 5, 5
    dec.reset()
    dec.forward_hidden([50258, 50259, 50359], hid[:3], stream)
    beams = [dec] + [dec.fork(stream) for _ in range(nb - 1)]
    hb = torch.empty(nb, d, device="cuda:0")
    lb = torch.empty(nb, vocab, device="cuda:0")
    ids = torch.empty(nb, k, dtype=torch.int32, device="cuda:0")
    lps = torch.empty(nb, k, device="cuda:0")
    toks = [440, 3111, 50257, 13, 1029]

    def beam_step():
        A.decoder_forward_beams(beams, toks, hb, stream)
        emb.matmul_dev(hb, nb, lb, stream=stream)
        A.logits_topk_dev(lb, nb, vocab, k, ids, lps, stream)

    beam_step()  # warm
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        beam_step()
    e1.record()
    torch.cuda.synchronize()
    beam_ms = e0.elapsed_time(e1) / steps
    ok = ok and bool(torch.isfinite(lps).all().item())
    t0 = time.perf_counter()
    extra = [beams[1].fork(stream) for _ in range(4)]
    torch.cuda.synchronize()
    fork_ms = (time.perf_counter() - t0) * 1e3 / 4
    for b in extra + beams[1:]:
        b.free()
    dec.free()
    return t_audio, per_len, ok, {"beams": nb, "ms_per_step": beam_ms, "cache_rows": f"5..{4 + steps}",
                                  "fork_ms": fork_ms}


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


def cpu_description():
    """The host CPU: model name, and the logical and physical cores this
    process may run on (its affinity mask)."""
    allowed = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else set(range(os.cpu_count() or 1))
    model, phys = "", set()
    try:
        for block in open("/proc/cpuinfo").read().split("\n\n"):
            f = dict(line.split(":", 1) for line in block.splitlines() if ":" in line)
            f = {k.strip(): v.strip() for k, v in f.items()}
            if "processor" not in f or int(f["processor"]) not in allowed:
                continue
            model = model or f.get("model name", "")
            phys.add((f.get("physical id", "0"), f.get("core id", f["processor"])))
    except OSError:
        pass
    return {"cpu_model": model, "logical_cores": len(allowed), "physical_cores": len(phys) or None}


def cpu_threads():
    import oracle as O

    threads = O.cpu_threads()
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit():
        threads = min(threads, int(cap))
    return threads


def cpu_baseline(synth, dtype: int, m: int, budget_s: float):
    """The reference CPU path (oracle/cpu_baseline.c) on one large-v3 encoder
    layer: each of the six linears on its first call (cold path, as the
    encoder runs in production), median of repeated runs."""
    import numpy as np

    import oracle as O

    cfg = synth.LARGE_V3
    shapes = synth.encoder_layer_shapes(cfg["d"], cfg["fc"])
    threads = cpu_threads()
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
    return dict({
        "value": round(ops / layer_s / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"one large-v3 encoder layer (6 {synth.NAMES[dtype]} linears, M={m}), cold path, median of {reps} "
                  f"runs per linear, tier {tier_name}, {threads} threads",
        "layer_ms": round(layer_s * 1e3, 2),
    }, **cpu_description())


def cpu_baseline_decode(synth, dtype: int, m: int, budget_s: float):
    """The reference CPU path on the decoder shapes at steady state: one
    large-v3 decoder layer's ten linears and the logits projection, each
    timed from its third call on (the packed int8 cache, src/quant.rs:589-639),
    median of repeated runs; the set's time is 32 layers plus the logits."""
    import numpy as np

    import oracle as O

    cfg = synth.LARGE_V3
    d, fc, vocab = cfg["d"], cfg["fc"], cfg["n_vocab"]
    shapes = synth.decoder_layer_shapes(d, fc) + [("logits", vocab, d)]
    threads = cpu_threads()
    rng = np.random.default_rng(8)
    times = []
    t_start = time.time()
    for i, (_, n, k) in enumerate(shapes):
        t = O.CpuQTensor(dtype, n, k, synth.normal_weights(dtype, n, k, seed=950 + i))
        a = rng.standard_normal((m, k)).astype(np.float32)
        t.matmul(a, threads=threads)
        t.matmul(a, threads=threads)  # the second call builds the packed cache
        runs = []
        while len(runs) < 5 or (len(runs) < 50 and time.time() - t_start < budget_s * (i + 1) / len(shapes)):
            t0 = time.perf_counter()
            t.matmul(a, threads=threads)
            runs.append(time.perf_counter() - t0)
        times.append(statistics.median(runs))
        t.close()
    set_s = cfg["layers"] * sum(times[:-1]) + times[-1]
    wbytes = sum(n * (k // 32) * synth.BLOCK_BYTES[dtype] for _, n, k in shapes[:-1]) * cfg["layers"] + \
        vocab * (d // 32) * synth.BLOCK_BYTES[dtype]
    io = cfg["layers"] * sum(4 * m * (n + k) for _, n, k in shapes[:-1]) + 4 * m * (vocab + d)
    return {
        "value": round((wbytes + io) / set_s / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"one large-v3 decoder layer's 10 {synth.NAMES[dtype]} linears and the [51866x1280] logits at "
                  f"M={m}, packed cache (third call on), median of >= 5 runs each; set = 32 layers + logits",
        "set_ms": round(set_s * 1e3, 3),
        "layer_ms": round(sum(times[:-1]) * 1e3, 3),
        "logits_ms": round(times[-1] * 1e3, 3),
    }


def leg_encoder(A, synth, torch, dtype: int, m: int, steps: int, warmup: int, seed0: int, cfg=None,
                spread: bool = False, outliers: float = 0.0, layers_w=None, name: str = ""):
    """One encoder-linears step of a configuration (graph replay)."""
    W = encoder_workload(A, synth, torch, dtype, m, seed0, cfg=cfg, spread=spread, outliers=outliers,
                         layers_w=layers_w)
    ms = time_encoder_graph(A, torch, W, steps, warmup)
    tops = W["ops"] / (ms * 1e-3) / 1e12
    cfg = cfg or synth.LARGE_V3
    log(f"{name}: {ms:.3f} ms per step ({tops:.1f} TOPS)")
    res = {"workload": f"{cfg['layers']} encoder layers' linears (d={cfg['d']}, fc {cfg['fc']}), "
                       f"{synth.NAMES[dtype]}, M={m}" + (", block scales spread 10**U(-1,1)" if spread else "")
                       + (f", {outliers:.0%} of input channels x20" if outliers else ""),
           "value": round(tops, 3), "unit": "TOPS", "ms_per_step": round(ms, 4), "peak": F16_PEAK_TFLOPS,
           "frac": round(tops / F16_PEAK_TFLOPS, 4), "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
    return res, W


def leg_single(A, synth, torch, dtype: int, n: int, k: int, m: int, steps: int, seed: int):
    """One matmul_t_q call (quantize + product) on resident inputs, 20 calls
    per graph replay."""
    dev = "cuda:0"
    w = A.DeviceWeight(dtype, n, k, synth.normal_weights(dtype, n, k, seed=seed))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn(m, k, device=dev, generator=g)
    b = torch.randn(n, device=dev, generator=g) * 0.1
    o = torch.empty(m, n, device=dev)
    wsz = A.workspace_size(m, k)
    ws = torch.empty(wsz, dtype=torch.uint8, device=dev)
    reps = 20
    ms = time_graph(torch, lambda st: [w.matmul_dev(a, m, o, b, ws, wsz, st) for _ in range(reps)], steps, 2) / reps
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    w.free()
    return {"workload": f"one {synth.NAMES[dtype]} matmul_t_q [{m}x{k}] x [{n}x{k}]^T + bias, quantization "
                        f"included", "value": round(tops, 3), "unit": "TOPS", "us_per_call": round(ms * 1e3, 2),
            "peak": F16_PEAK_TFLOPS, "frac": round(tops / F16_PEAK_TFLOPS, 4)}


def leg_turbo_decoder(A, synth, torch, layers_w, steps: int, seed0: int):
    """large-v3-turbo's 4-layer decoder over 8 stacked windows, Q5_1: the
    cross K/V projections of the 8 x 1500 encoder rows (once per window
    batch), then per step the 8 per-token linears of every layer and the
    logits at M = 8 x 5 beam rows (quantization + product per linear)."""
    dev = "cuda:0"
    dtype, d, fc, vocab, nl = synth.BY_NAME["Q5_1"], 1280, 5120, 51866, 4
    g = torch.Generator(device=dev)
    g.manual_seed(seed0)
    # cross K/V: the encoder's q/k weights stand in (same shapes and dtype)
    M = 8 * 1500
    enc = torch.randn(M, d, device=dev, generator=g)
    kv = [[torch.empty(M, d, device=dev) for _ in range(2)] for _ in range(nl)]
    kv_b = torch.randn(d, device=dev, generator=g) * 0.1
    wsz = A.workspace_size(M, d)
    ws = torch.empty(wsz, dtype=torch.uint8, device=dev)

    def cross(st):
        A.quantize_dev(enc, M, d, ws, wsz, st)
        for l in range(nl):
            A.matmul_prequant_multi_dev([layers_w[l]["q"], layers_w[l]["k"]], ws, M, kv[l], [None, kv_b], st)

    ms_cross = time_graph(torch, cross, max(2, steps // 2), 1)
    ops_cross = nl * 2 * 2 * M * d * d
    # per-token linears at m = 40
    m = 40
    per = [("q", d, d), ("k", d, d), ("v", d, d), ("out", d, d), ("cq", d, d), ("cout", d, d), ("fc1", fc, d),
           ("fc2", d, fc)]
    raws = synth.normal_weights_many([(dtype, n, k, seed0 + i) for i, (_, n, k) in enumerate(per * nl)]
                                     + [(dtype, vocab, d, seed0 + 99)], min(16, os.cpu_count() or 1))
    ws_ = [A.DeviceWeight(dtype, n, k, r) for (_, n, k), r in zip(per * nl + [("logits", vocab, d)], raws)]
    ins = [torch.randn(m, w.k, device=dev, generator=g) for w in ws_]
    outs = [torch.empty(m, w.n, device=dev) for w in ws_]
    bs = [None if i % 8 == 1 or i == len(ws_) - 1 else torch.randn(w.n, device=dev, generator=g) * 0.1
          for i, w in enumerate(ws_)]
    wk = {k: (A.workspace_size(m, k), torch.empty(A.workspace_size(m, k), dtype=torch.uint8, device=dev))
          for k in (d, fc)}

    def step(st):
        for w, a, o, b in zip(ws_, ins, outs, bs):
            w.matmul_dev(a, m, o, b, wk[w.k][1], wk[w.k][0], st)

    ms_step = time_graph(torch, step, steps, 2)
    ops_step = sum(2 * m * w.n * w.k for w in ws_)
    wbytes = sum(w.n * (w.k // 32) * synth.BLOCK_BYTES[dtype] for w in ws_)
    # the prompt's prefill: the same per-layer linears at M = 224 prompt rows
    # (no logits; src/transcribe.rs:540-561 runs prompts of up to 224 tokens)
    mp = 224
    lin = ws_[:-1]
    ins_p = [torch.randn(mp, w.k, device=dev, generator=g) for w in lin]
    outs_p = [torch.empty(mp, w.n, device=dev) for w in lin]
    wk_p = {k: (A.workspace_size(mp, k), torch.empty(A.workspace_size(mp, k), dtype=torch.uint8, device=dev))
            for k in (d, fc)}

    def prefill(st):
        for w, a, o, b in zip(lin, ins_p, outs_p, bs):
            w.matmul_dev(a, mp, o, b, wk_p[w.k][1], wk_p[w.k][0], st)

    ms_pre = time_graph(torch, prefill, steps, 2)
    ops_pre = sum(2 * mp * w.n * w.k for w in lin)
    for w in ws_:
        w.free()
    return {
        "cross_kv": {"workload": "cross-attention K and V of 4 decoder layers over 8 stacked windows (M=12000, "
                                 "1280x1280 Q5_1): one quantization, one two-weight GEMM launch per layer",
                     "value": round(ops_cross / (ms_cross * 1e-3) / 1e12, 3), "unit": "TOPS",
                     "ms": round(ms_cross, 4)},
        "step_m40": {"workload": "per decoder step at M=40 (8 windows x 5 beams): 4 layers x (self q,k,v,out, "
                                 "cross q,out, fc1, fc2) + logits [51866x1280], Q5_1, each a quantization and a "
                                 "64-row-tile GEMM launch",
                     "value": round(ops_step / (ms_step * 1e-3) / 1e12, 3), "unit": "TOPS",
                     "ms": round(ms_step, 4),
                     "weight_GB_per_s": round(wbytes / (ms_step * 1e-3) / 1e9, 1)},
        "prefill_m224": {"workload": "prompt prefill at M=224: 4 layers x (self q,k,v,out, cross q,out, fc1, fc2), "
                                     "Q5_1, each a quantization and a GEMM launch",
                         "value": round(ops_pre / (ms_pre * 1e-3) / 1e12, 3), "unit": "TOPS",
                         "ms": round(ms_pre, 4)},
    }


def leg_host_entry(A, W, D, reps: int = 5):
    """The drop-in entry itself, rw_rocm_matmul_t_q (what linear_w / matmul_t_q
    routes to, src/quant.rs:754,1054-1063): host arrays in and out, pageable
    as a Rust Vec<f32> is; per call the activation and bias go to the device,
    the activation is quantized, the product runs and the output comes back,
    synchronously.  Encoder: layer 0's six linears at M = W["m"]; decode: one
    decoder layer's ten linears plus the logits at M = D["rows"].  Host wall
    clock, median of `reps` passes after one warm pass."""
    import numpy as np

    rng = np.random.default_rng(17)

    def run(calls):
        times = []
        for it in range(reps + 1):
            t0 = time.perf_counter()
            for w, a, b in calls:
                w.matmul(a, b)
            if it:
                times.append(time.perf_counter() - t0)
        return statistics.median(times) * 1e3

    m = W["m"]
    lw = W["layers"][0]
    enc = [(lw[name], rng.standard_normal((m, k), dtype=np.float32),
            None if W["bias"][name] is None else W["bias"][name].cpu().numpy()) for name, n, k in W["shapes"]]
    ems = run(enc)
    eops = sum(2 * m * w.n * w.k for w, _, _ in enc)
    epcie = sum(4 * m * (w.k + w.n) for w, _, _ in enc)
    md = D["rows"]
    dsel = list(D["items"][:10]) + [D["items"][-1]]
    dec = [(w, rng.standard_normal((md, w.k), dtype=np.float32), None if b is None else b.cpu().numpy())
           for (w, _, b, _, _) in dsel]
    dms = run(dec)
    dbytes = sum(w.n * (w.k // 32) * A.block_bytes(w.dtype) + 4 * md * (w.k + w.n) for w, _, _ in dec)
    return {
        "workload": "rw_rocm_matmul_t_q with pageable host arrays (PCIe copies, quantization and product per "
                    f"call, synchronous): encoder = large-v3 layer 0's six linears at M={m}; decode = one large-v3 "
                    f"decoder layer's ten linears plus the [51866 x 1280] logits at M={md}",
        "encoder_ms_per_layer": round(ems, 3),
        "encoder_TOPS": round(eops / (ems * 1e-3) / 1e12, 3),
        "encoder_pcie_bytes": epcie,
        "decode_ms_per_layer_and_logits": round(dms, 3),
        "decode_GB_per_s": round(dbytes / (dms * 1e-3) / 1e9, 2),
        "decode_calls": len(dec),
        "note": "host wall clock around synchronous calls; the device-resident figures are the _dev entries",
    }


def profile_traffic(root: str):
    """HBM bytes per k_gemm launch of the headline workload, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (the json block of
    profiles/k_gemm_q5_1_large_v3_encoder_m1500.md); None when absent."""
    path = os.path.join(root, "profiles", "k_gemm_q5_1_large_v3_encoder_m1500.md")
    try:
        text = open(path).read()
        blob = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(blob), os.path.relpath(path, root)
    except (OSError, IndexError, ValueError):
        return None, None


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
    ap.add_argument("--no-legs", action="store_true", help="skip the other configurations' legs")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--no-host-entry", action="store_true", help="skip timing rw_rocm_matmul_t_q on host arrays")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="skip the per-launch k_gemm bursts (graph replays), e.g. under a counter profiler")
    ap.add_argument("--eager", action="store_true",
                    help="report the eager step (no graph capture), e.g. under a counter profiler")
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
    ms = eager_ms if args.eager else time_encoder_graph(A, torch, W, args.steps, args.warmup)
    tops = W["ops"] / (ms * 1e-3) / 1e12
    log(f"encoder step, {'eager' if args.eager else 'graph replay'} {ms:.3f} ms  ({tops:.1f} TOPS)")
    fms = None
    if not args.eager:
        fms = time_encoder_graph(A, torch, W, args.steps, args.warmup, fused=True)
        log(f"encoder step with the MLP as the encoder runs it (fc2 on gelu(fc1), quantized in fc1's epilogue): "
            f"{fms:.3f} ms ({W['ops'] / (fms * 1e-3) / 1e12:.1f} TOPS)")

    if args.no_kernel_timing:
        gemm_ms, gemm_ops, launches, per_shape = ms / (4 * len(W["layers"])), W["ops"] / (4 * len(W["layers"])), 0, {}
    else:
        gemm_ms, gemm_ops, launches, per_shape = time_gemm_kernel(A, torch, W, stream)
    gemm_tops = gemm_ops / (gemm_ms * 1e-3) / 1e12
    log(f"k_gemm average launch {gemm_ms * 1e3:.1f} us over {launches} launches -> {gemm_tops:.1f} TOPS "
        f"(per launch, us: {per_shape})")
    prof, prof_path = profile_traffic(ROOT)
    traffic = None
    if prof and args.quant == "Q5_1" and args.m == 1500:
        # the same launch mix as `achieved`: one of each launch type per layer
        traffic = int(sum(prof["fetch_bytes"][k] + prof["write_bytes"][k] for k, _ in LAUNCHES) / len(LAUNCHES))

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
        "fused_mlp": None if fms is None else {
            "ms_per_step": round(fms, 4),
            "TOPS": round(W["ops"] / (fms * 1e-3) / 1e12, 3),
            "workload": "the same step with fc2's input gelu(fc1's output), as the encoder's MLP runs "
                        "(src/encoder.rs:161-171): fc1's epilogue adds the bias, applies GELU and quantizes "
                        "for fc2 (rw_rocm_matmul_prequant_gelu_quantize_dev), so the step has 3 quantizations and "
                        "does the GELU work the headline step does not"},
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
            "traffic": traffic,
            "traffic_source": prof_path if traffic is not None else None,
            "kernel": f"k_gemm<{args.quant}> on v_mfma_f32_32x32x16_f16 (2*M*N*K per launch)",
            "limiter": "operand delivery at one wavefront per SIMD (the k loop takes the MFMA-only loop plus "
                       "35-50% of the loads-only one), and every wavefront waiting for its first blocks and "
                       "storing its tile at once: MFMA busy about a quarter of the kernel's time, L2->CU operand "
                       "traffic 10-25x the unique bytes (rocprofv3 counters in "
                       "profiles/k_gemm_q5_1_large_v3_encoder_m1500.md)",
            "avg_launch_us": round(gemm_ms * 1e3, 2),
            "launch_us_by_launch": per_shape,
            "frac_of_int8_peak": round(gemm_tops / INT8_PEAK_TOPS, 4),
        },
    }
    if not args.no_cold:
        Wc = encoder_workload(A, synth, torch, dtype, args.m, seed0=1, layers_w=W["layers"], cold=True)
        cms = time_encoder_graph(A, torch, Wc, max(3, args.steps // 2), 1)
        ctops = W["ops"] / (cms * 1e-3) / 1e12
        log(f"encoder step, cold (every layer its own buffers): {cms:.3f} ms ({ctops:.1f} TOPS)")
        result["cold"] = {"workload": "the headline step with every layer's inputs, outputs and workspaces its "
                                      "own (2.6 GB of buffers, more than ten MALLs), graph replay",
                          "value": round(ctops, 3), "unit": "TOPS", "ms_per_step": round(cms, 4)}
        del Wc
        torch.cuda.empty_cache()
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

    legs = {}
    if not args.no_legs:
        steps = max(3, args.steps // 2)
        legs["c1_tiny_fc1_q5_1"] = leg_single(A, synth, torch, synth.BY_NAME["Q5_1"], 1536, 384, 1500, steps, 43)
        log(f"tiny.en fc1: {legs['c1_tiny_fc1_q5_1']['us_per_call']} us per call "
            f"({legs['c1_tiny_fc1_q5_1']['value']} TOPS)")
        legs["c2_small_encoder_q8_0"], _ = leg_encoder(A, synth, torch, synth.BY_NAME["Q8_0"], 1500, steps, 1, 2,
                                                       cfg=synth.SMALL, outliers=0.01, name="small.en Q8_0")
        for q in ("Q4_0", "Q4_1"):
            legs[f"c4_large_v3_encoder_{q.lower()}"], Wq = leg_encoder(A, synth, torch, synth.BY_NAME[q], 1500,
                                                                      steps, 1, 4, spread=True,
                                                                      name=f"large-v3 {q} spread")
            del Wq
            torch.cuda.empty_cache()
        legs["c5_turbo_encoder_m12000_q5_1"], Wt = leg_encoder(A, synth, torch, dtype, 12000, 2, 1, 5,
                                                               layers_w=W["layers"], name="turbo M=12000")
        if not args.no_kernel_timing:
            # k_gemm alone at M = 12000: the same per-launch-type bursts as the headline's
            t_ms, t_ops, _, t_per = time_gemm_kernel(A, torch, Wt, stream, reps=1)
            legs["c5_turbo_encoder_m12000_q5_1"]["k_gemm"] = {
                "avg_launch_us": round(t_ms * 1e3, 2), "TFLOP_per_s": round(t_ops / (t_ms * 1e-3) / 1e12, 1),
                "launch_us_by_launch": t_per,
                "note": "per launch type, the 32 layers' launches back to back in a replayed HIP graph"}
            log(f"turbo M=12000 k_gemm: {t_ms * 1e3:.1f} us average launch, {t_per}")
        del Wt
        torch.cuda.empty_cache()
        t = leg_turbo_decoder(A, synth, torch, W["layers"], steps, 6)
        legs["c5_turbo_cross_kv_m12000_q5_1"] = t["cross_kv"]
        legs["c5_turbo_decoder_m40_q5_1"] = t["step_m40"]
        legs["c5_turbo_prefill_m224_q5_1"] = t["prefill_m224"]
        log(f"turbo cross K/V {t['cross_kv']['ms']} ms ({t['cross_kv']['value']} TOPS); M=40 step "
            f"{t['step_m40']['ms']} ms ({t['step_m40']['value']} TOPS); prefill M=224 "
            f"{t['prefill_m224']['ms']} ms ({t['prefill_m224']['value']} TOPS)")
        torch.cuda.empty_cache()

    W_host = None if args.no_host_entry else {k: W[k] for k in ("layers", "shapes", "bias", "m")}
    W_host = W_host and dict(W_host, layers=W["layers"][:1])
    del W
    torch.cuda.empty_cache()

    if not args.no_decode:
        D = decode_workload(A, synth, torch, synth.BY_NAME[args.decode_quant], args.decode_m, seed0=5000)
        dms, dms_call = time_decode(A, torch, D, max(3, args.steps), 2, stream)
        gbs = D["bytes"] / (dms * 1e-3) / 1e9
        log(f"decode set M={args.decode_m}: {dms:.3f} ms ({gbs:.1f} GB/s); with per-call table upload "
            f"{dms_call:.3f} ms")
        result["decode"] = {
            "metric": f"decode GEMV HBM GB/s @M={args.decode_m}",
            "workload": f"large-v3 decoder linears, {args.decode_quant}, M={args.decode_m}: 32 layers x 10 "
                        f"linears + logits [51866x1280], {D['count']} independent linears per step",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(dms, 4),
            "ms_per_step_with_table_upload": round(dms_call, 4),
            "bytes_per_step": D["bytes"],
            "launch": "prepared group (rw_rocm_group_run): one k_gemv_records launch (each linear's activation "
                      "quantized once) and one k_gemv launch for the set",
            "peak": HBM_PEAK_GBS,
            "frac": round(gbs / HBM_PEAK_GBS, 4),
        }
        if args.decode_m > 1:
            D1 = decode_rows(A, torch, D, 1)
            d1, _ = time_decode(A, torch, D1, max(3, args.steps), 2, stream)
            g1 = D1["bytes"] / (d1 * 1e-3) / 1e9
            log(f"decode set M=1: {d1:.3f} ms ({g1:.1f} GB/s)")
            legs["c3_decode_m1_" + args.decode_quant.lower()] = {
                "workload": f"the decode set at M=1 (greedy), {args.decode_quant}", "value": round(g1, 2),
                "unit": "GB/s", "ms_per_step": round(d1, 4), "bytes_per_step": D1["bytes"],
                "peak": HBM_PEAK_GBS, "frac": round(g1 / HBM_PEAK_GBS, 4)}
            del D1
        if not args.no_layers:
            t_audio, per_len, finite, beam = time_decoder_tokens(A, synth, torch, D, stream, 20)
            log(f"decoder on the device: set_audio {t_audio['warm_ms']:.3f} ms warm ({t_audio['cold_ms']:.2f} ms "
                f"first call), ms per token with logits by cache length "
                f"{ {k: round(v, 3) for k, v in per_len.items()} } (finite={finite})")
            result["decoder_tokens"] = {
                "workload": "large-v3 decoder, one beam, Q5_0: per token the embedding, 32 layers (causal "
                            "self-attention over the cache, cross-attention to 1500 positions, MLP), final "
                            "layernorm and the [51866 x 1280] logits product, all on the device (rw_decoder)",
                "ms_per_token": round(per_len[24], 4),
                "ms_per_token_by_cache_length": {str(k): round(v, 4) for k, v in per_len.items()},
                "note": "ms_per_token: steps 5..24 of the cache (3-token prompt, one warm step, 20 timed); the "
                        "other lengths time 4 steps ending at that many cached rows",
                "set_audio_ms": round(t_audio["warm_ms"], 3),
                "set_audio_first_call_ms": round(t_audio["cold_ms"], 3),
                "set_audio_note": "set_audio_ms: median of 7 later calls (HIP events on the launching stream); "
                                  "the first call also allocates the decoder's workspace (host clock)",
                "finite": finite,
                "beams": {
                    "workload": f"beam search step, {beam['beams']} beams forked from one decoder: "
                                "rw_rocm_decoder_forward_beams_dev (every linear over the 5 rows, the beams' "
                                "self-attentions in one launch), the stacked [5 x 51866] logits product, and "
                                "log_softmax + top-5 per beam on the device (rw_rocm_logits_topk_dev)",
                    "ms_per_step": round(beam["ms_per_step"], 4),
                    "ms_per_token_per_beam": round(beam["ms_per_step"] / beam["beams"], 4),
                    "cache_rows": beam["cache_rows"],
                    "fork_ms": round(beam["fork_ms"], 3),
                    "note": "fork_ms: one rw_rocm_decoder_fork at 24 cached rows (the beam search forks the "
                            "surviving candidates every step), host wall time",
                },
            }
            log(f"beam step ({beam['beams']} beams): {beam['ms_per_step']:.3f} ms, "
                f"{beam['ms_per_step'] / beam['beams']:.3f} ms per token per beam; fork {beam['fork_ms']:.3f} ms")
        if W_host is not None:
            h = leg_host_entry(A, W_host, D)
            log(f"host entry rw_rocm_matmul_t_q: encoder layer {h['encoder_ms_per_layer']} ms "
                f"({h['encoder_TOPS']} TOPS), decoder layer + logits {h['decode_ms_per_layer_and_logits']} ms "
                f"({h['decode_GB_per_s']} GB/s)")
            result["host_entry"] = h
        del D
        torch.cuda.empty_cache()
    if legs:
        result["legs"] = legs

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
        log(f"cpu baseline {cb['value']} TOPS ({cb['sample']}; {cb['cpu_model']})")
        cd = cpu_baseline_decode(synth, synth.BY_NAME[args.decode_quant], args.decode_m, args.cpu_seconds)
        log(f"cpu baseline, decoder shapes {cd['value']} GB/s ({cd['sample']})")
        cb["decode"] = cd
        result["cpu_baseline"] = cb

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
