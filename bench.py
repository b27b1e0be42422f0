#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: Q4_0 decode GEMV with the FFN gate/up
shape, N = 14336 rows x K = 4096, f32 activations, as woolly's
simd::quantized_matvec computes it.  One step = one GEMV launch over one
weight matrix already resident in HBM.  The timed loop rotates through 10
distinct weight copies (10 x 33 MB = 330 MB, more than the 256 MB Infinity
Cache), so every launch streams its weights from HBM.

Prints ONE JSON line with:
  value          algorithmic GB/s of the GEMV = bytes per launch / ms_per_step,
                 bytes = N*K/32*18 (weights) + 4K (x) + 4N (y) = 33,103,872 B
  roofline       the GEMV kernel's average launch duration against the 8 TB/s HBM
                 peak: the K launches are captured into one HIP graph, which is
                 replayed back to back between two HIP events on the launch
                 stream (at least 1000 launches per measurement, so a short
                 graph's per-replay cost stays hidden), median of 5 measurements
                 after ~0.1 s of clock settling; traffic = HBM bytes per launch
                 from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary,
                 null when that summary was taken from other kernel sources;
                 read_floor: the same bytes read by wh_read_probe in the GEMV's
                 workgroup geometry with no compute, timed the same way (what one
                 launch of this access pattern reaches on this part), and as one
                 flat range with every load in flight at once (what one launch
                 reading these bytes reaches); launch_us_eager_*: the same GEMV
                 launched one call at a time without a graph
  ffn_layer_us   the fused SwiGLU FFN layer (Llama-3-8B shape, Q4_0) at M=1, 2, 4
                 and 512, same run (the metric's second part; M <= 16 rotates
                 3 layers' weights, 297 MB, past the Infinity Cache)
  every leg      graph replays between events on the launch stream after ~0.1 s
                 of clock settling, median of 5 measurements of >= 10 ms each;
                 "spread" = (max - min) / median of the 5
  host_slice_*   the synchronous host-slice drop-in on the headline matrix: wall
                 µs per call uploading the weights each call, and with the device
                 copies of host weights on
  prefill_*      config 2's M sweep (f32 and bf16 activations); the K-quant
                 formats and Q4_1 at a few tokens, and at M=512 with blocks
                 converted once per weight handle (and, for comparison, per call);
                 Q4_1's GEMM and FFN at M=512
  gemv_other_configs  the other decode GEMV configurations: Q4_0 4096x4096,
                 Q8_0 and Q4_1 14336x4096, and the other decode-step shapes (k/v
                 projections, FFN down, the Q8_0 128256x4096 output head):
                 µs, algorithmic GB/s, fraction of peak
  decode_step_llama3_8b_q4_0  config 4: one decode step (32 Q4_0 layers,
                 Q8_0 head, f16 KV cache at context 4096) replayed as one HIP graph:
                 tokens/s and algorithmic GB/s (weights + KV cache read once)
  cpu_baseline   the reference's intended SIMD GEMV (8-lane AVX2 FMA, restated in
                 the test oracle) on up to 16 host threads, a bounded sample of
                 full-size calls; cpu_baseline_scalar: the order-exact scalar
                 quantized_matvec_q4_0_scalar on 1 thread
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_0 GEMV achieved HBM GB/s (% of peak); FFN-layer µs at M=1 and M=512"
Q4_0 = 2
N_ROWS, K = 14336, 4096
REPLICAS = 10
WARM_S = 0.1          # untimed replays before each leg's timed measurements (clock settling)
TIMED_REPLAYS = 5     # timed measurements per leg; the median is reported, with the spread
TIMED_LAUNCHES = 1000  # GEMV: launches per measurement (back-to-back replays of the K-launch graph)
MIN_MEASURE_MS = 10.0  # every leg: a measurement lasts at least this long


TYPE_SIZE = {2: 18, 3: 20, 8: 34, 12: 144, 14: 210}
BLOCK_ELEMS = {2: 32, 3: 32, 8: 32, 12: 256, 14: 256}


def gemv_bytes(n: int, k: int, t: int = Q4_0) -> int:
    return n * (k // BLOCK_ELEMS[t]) * TYPE_SIZE[t] + 4 * k + 4 * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_graph(run, n_calls: int, stream, min_launches: int = 1) -> tuple[float, float]:
    """The timing every leg shares: run(i) for i < n_calls is captured once
    into a HIP graph; one replay does the first-launch setup, untimed replays
    run the GPU for WARM_S seconds (its clocks settle), then TIMED_REPLAYS
    measurements each time back-to-back replays of the graph between two
    events on the launch stream (at least min_launches calls and
    MIN_MEASURE_MS per measurement, so the per-replay cost of a short graph
    stays hidden behind the previous replay's kernels).  Returns (median ms
    per call, spread = (max - min) / median of the measurements)."""
    from woolly_amd.device import Event, Graph

    with Graph.capture(stream) as graph:
        for i in range(n_calls):
            run(i)
    e0, e1 = Event(), Event()
    e0.record(stream)
    graph.launch(stream)  # first-launch setup
    e1.record(stream)
    e1.synchronize()
    first_ms = max(e0.elapsed_ms(e1), 1e-3)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARM_S:
        graph.launch(stream)
        stream.synchronize()
    n_rep = max(1, -(-min_launches // n_calls), int(np.ceil(MIN_MEASURE_MS / first_ms)))
    reps = []
    for _ in range(TIMED_REPLAYS):
        e0.record(stream)
        for _ in range(n_rep):
            graph.launch(stream)
        e1.record(stream)
        e1.synchronize()
        reps.append(e0.elapsed_ms(e1) / (n_rep * n_calls))
    graph.destroy()
    e0.destroy()
    e1.destroy()
    med = float(np.median(reps))
    time_graph.calls_timed = n_rep * n_calls
    return med, (max(reps) - min(reps)) / med


def bench_gemv(steps: int, warmup: int, t: int = Q4_0, n: int = N_ROWS, k: int = K, seed: int = 3,
               replicas: int = REPLICAS):
    """GEMV y = W x of type t, n x k: (ms per launch over a graph replay of
    `steps` launches, median and mean of event-bracketed eager launches).
    `replicas` weight copies are rotated so the weights come from HBM."""
    from woolly_amd import ops, synth
    from woolly_amd.device import DeviceBuffer, Event, Graph, Stream

    w = synth.quantized_weight(t, n, k, seed=seed)
    x = synth.activations(k, seed=seed)
    stream = Stream()
    wbufs = [DeviceBuffer.from_array(w) for _ in range(replicas)]
    xb = DeviceBuffer.from_array(x)
    yb = DeviceBuffer(4 * n)

    def launch(i: int) -> None:
        ops.quantized_matvec(t, wbufs[i % replicas], w.nbytes, xb, yb, n, k, stream)

    for i in range(warmup):
        launch(i)
    stream.synchronize()

    # The K timed launches are captured once into a HIP graph and replayed, so
    # the host's per-call overhead does not throttle the GPU (at least
    # TIMED_LAUNCHES launches per measurement, median of TIMED_REPLAYS)
    ms_per, spread = time_graph(launch, steps, stream, TIMED_LAUNCHES)
    bench_gemv.launches_timed = time_graph.calls_timed
    bench_gemv.spread = spread

    # eager launches (no graph), as a caller launching one call at a time sees
    # them: 200 back-to-back calls between two events, and an event pair
    # around each of 200 calls
    n_eager = 200
    e0, e1 = Event(), Event()
    for i in range(20):
        launch(i)
    e0.record(stream)
    for i in range(n_eager):
        launch(i)
    e1.record(stream)
    e1.synchronize()
    bench_gemv.eager_back_to_back_ms = e0.elapsed_ms(e1) / n_eager
    e0.destroy()
    e1.destroy()
    n_pairs = min(steps, 200)
    evs = [(Event(), Event()) for _ in range(n_pairs)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        launch(i)
        b.record(stream)
    stream.synchronize()
    durs = np.array([a.elapsed_ms(b) for a, b in evs])
    for a, b in evs:
        a.destroy()
        b.destroy()
    return ms_per, float(np.median(durs)), float(np.mean(durs))


def bench_ffn(m: int, iters: int, t: int = Q4_0, replicas: int | None = None,
              prepared: bool = False) -> tuple[float, float]:
    """The SwiGLU FFN layer (config 3, Llama-3-8B shape), (µs per call,
    spread).  The weights of `replicas` layers (default: enough copies for
    > 256 MB, the Infinity Cache, when the call streams its weights once,
    M <= 16) are rotated; the calls are captured into a HIP graph and replayed
    (time_graph).  prepared: the weights are wh_weight handles whose K-quant
    blocks were converted once for prefill (wh_weight_prepare_prefill)."""
    from woolly_amd import ops, synth
    from woolly_amd.device import DeviceBuffer, Stream

    hidden, n_ff = 4096, 14336
    L = synth.ffn_layer(t, hidden, n_ff, m, seed=5)
    wbytes = L["gate"].nbytes + L["up"].nbytes + L["down"].nbytes
    if replicas is None:
        replicas = max(1, -(-300_000_000 // wbytes)) if m <= 16 else 1
    stream = Stream()
    if prepared:
        shapes = {"gate": (n_ff, hidden), "up": (n_ff, hidden), "down": (hidden, n_ff)}
        copies = [{k: ops.Weight(t, *shapes[k], L[k]) for k in shapes} for _ in range(replicas)]
        for c in copies:
            for w in c.values():
                w.prepare_prefill(stream)
        ptrs = [{k: w.ptr for k, w in c.items()} for c in copies]
    else:
        copies = [{k: DeviceBuffer.from_array(L[k]) for k in ("gate", "up", "down")} for _ in range(replicas)]
        ptrs = copies
    b = {k: DeviceBuffer.from_array(L[k]) for k in ("gamma", "x")}
    out = DeviceBuffer(4 * m * hidden)
    wsz = ops.ffn_workspace_bytes(hidden, n_ff, m, ggml_type=t)
    ws = DeviceBuffer(wsz)

    def run(i):
        c = ptrs[i % replicas]
        ops.ffn_swiglu(t, c["gate"], c["up"], c["down"], hidden, n_ff, b["gamma"], 1e-5, b["x"],
                       m, out, ws, wsz, stream)

    for i in range(3):
        run(i)
    stream.synchronize()
    ms, spread = time_graph(run, max(iters, replicas), stream)
    return ms * 1000.0, spread


def bench_gemm(m: int, iters: int, t: int = Q4_0, bf16: bool = False, prepared: bool = False) -> tuple[float, float]:
    """Prefill GEMM Y[m, 14336] = X[m, 4096] W^T (config 2; Q4_0 unless t; X in
    bfloat16 with bf16), (µs per call, spread).  For m <= 64, where the call
    streams its 33 MB of weights about once, 10 weight copies (> 256 MB, the
    Infinity Cache) are rotated; the calls are captured into a HIP graph and
    replayed (time_graph).  prepared: the weights are wh_weight handles whose
    K-quant blocks were converted once for prefill."""
    from woolly_amd import ops, synth
    from woolly_amd.device import DeviceBuffer, Stream

    w = synth.quantized_weight(t, N_ROWS, K, seed=4)
    x = np.concatenate([synth.activations(K, seed=400 + i) for i in range(min(m, 64))])
    x = np.resize(x, m * K).astype(np.float32)
    if bf16:
        x = (x.view(np.uint32) >> 16).astype(np.uint16)
    replicas = 10 if m <= 64 else 1
    stream = Stream()
    if prepared:
        handles = [ops.Weight(t, N_ROWS, K, w) for _ in range(replicas)]
        for h in handles:
            h.prepare_prefill(stream)
        wbs = [h.ptr for h in handles]
    else:
        wbs = [DeviceBuffer.from_array(w) for _ in range(replicas)]
    xb = DeviceBuffer.from_array(x)
    yb = DeviceBuffer(4 * m * N_ROWS)
    wsz = (ops.matmul_x_workspace_bytes(t, N_ROWS, K, m, ops.TYPE_BF16) if bf16
           else ops.matmul_workspace_bytes(t, N_ROWS, K, m))
    ws = DeviceBuffer(max(wsz, 256))

    def run(i):
        if bf16:
            ops.quantized_matmul_x(t, wbs[i % replicas], w.nbytes, N_ROWS, K, xb, ops.TYPE_BF16, m, yb, ws, wsz,
                                   stream)
        else:
            ops.quantized_matmul(t, wbs[i % replicas], w.nbytes, N_ROWS, K, xb, m, yb, ws, wsz, stream)

    for i in range(3):
        run(i)
    stream.synchronize()
    ms, spread = time_graph(run, max(iters, replicas), stream)
    return ms * 1000.0, spread


# config 4: Llama-3-8B-shaped decode step
L8B = dict(hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, n_ff=14336, vocab=128256,
           n_layers=32, ctx=4096, rope_base=500000.0, eps=1e-5)


# per-matrix block types of a Q4_K_M file (attn_v and ffn_down in Q6_K, the
# other projections in Q4_K; its output head is Q6_K)
Q4_K_M = {"wq": 12, "wk": 12, "wv": 14, "wo": 12, "w_gate": 12, "w_up": 12, "w_down": 14}


def decode_shapes(c: dict) -> dict:
    h, nh, nkv, d, f = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["n_ff"]
    return {"wq": (nh * d, h), "wk": (nkv * d, h), "wv": (nkv * d, h), "wo": (h, nh * d),
            "w_gate": (f, h), "w_up": (f, h), "w_down": (h, f)}


def decode_bytes(c: dict = L8B, types: dict | None = None, head_type: int = 8) -> int:
    """Algorithmic HBM bytes of one decode step at context c['ctx']: every
    weight once, the whole KV cache of every layer once, norms, x and logits."""
    h, kv = c["hidden"], c["n_kv_heads"] * c["head_dim"]
    types = types or {k: Q4_0 for k in decode_shapes(c)}
    per_layer = sum(gemv_bytes(n, k, types[name]) - 4 * (n + k) for name, (n, k) in decode_shapes(c).items())
    per_layer += 2 * 4 * h
    kv_read = c["n_layers"] * 2 * c["ctx"] * kv * 2
    head = gemv_bytes(c["vocab"], h, head_type) - 4 * c["vocab"]
    return c["n_layers"] * per_layer + kv_read + head + 4 * h + 4 * c["vocab"]


def bench_decode(steps: int, c: dict = L8B, types: dict | None = None, head_type: int = 8) -> dict:
    """One decode step of a random-init 32-layer Llama-3-8B-shaped model (Q4_0
    matrices and a Q8_0 output head unless types / head_type say otherwise),
    f16 KV cache filled ~N(0,1), at position ctx - 1 (attention over ctx
    positions).  The step (all layers + head) is captured once into a HIP graph
    and replayed; returns timings."""
    from woolly_amd import ops, synth
    from woolly_amd.device import DeviceBuffer, Event, Graph, Stream

    h, nh, nkv, d, f = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["n_ff"]
    rng = np.random.default_rng(6)
    mats = decode_shapes(c)
    types = types or {k: Q4_0 for k in mats}
    # one layer's weights, uploaded to every layer's own buffers
    host = {k: synth.quantized_weight(types[k], n, kk, seed=60 + i) for i, (k, (n, kk)) in enumerate(mats.items())}
    kc = rng.standard_normal((c["ctx"], nkv, d)).astype(np.float16)
    vc = rng.standard_normal((c["ctx"], nkv, d)).astype(np.float16)
    layers = []
    for li in range(c["n_layers"]):
        L = {k: DeviceBuffer.from_array(v) for k, v in host.items()}
        L["attn_norm"] = DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(h)).astype(np.float32))
        L["ffn_norm"] = DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(h)).astype(np.float32))
        L["k_cache"] = DeviceBuffer.from_array(kc)
        L["v_cache"] = DeviceBuffer.from_array(vc)
        for k in mats:
            L[k + "_type"] = types[k]
        layers.append(L)
    # head: 1/8 of the rows generated, tiled into the full matrix
    part = synth.quantized_weight(head_type, c["vocab"] // 8, h, seed=70)
    head = DeviceBuffer(part.nbytes * 8)
    for i in range(8):
        head.upload(part, offset=i * part.nbytes)
    onorm = DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(h)).astype(np.float32))
    inv = DeviceBuffer.from_array(ops.rope_inv_freq(c["rope_base"], d))
    model = ops.LlamaModel(types["wq"], dict(hidden=h, n_heads=nh, n_kv_heads=nkv, head_dim=d, n_ff=f,
                                             max_ctx=c["ctx"], vocab=c["vocab"], eps=c["eps"]),
                           layers, inv, onorm, head, head_type)
    wsz = model.workspace_bytes()
    ws = DeviceBuffer(wsz)
    x0 = synth.activations(h, seed=6)
    xb, lb = DeviceBuffer.from_array(x0), DeviceBuffer(4 * c["vocab"])
    stream = Stream()
    pos = c["ctx"] - 1
    for _ in range(3):
        model.decode_step(pos, xb, lb, ws, wsz, stream)
    stream.synchronize()
    ms, spread = time_graph(lambda i: model.decode_step(pos, xb, lb, ws, wsz, stream), 1, stream, steps)
    logits = lb.download(np.float32, c["vocab"])
    nb = decode_bytes(c, types, head_type)
    return {"tokens_per_s": round(1000.0 / ms, 1), "ms_per_token": round(ms, 4), "bytes_per_token": nb,
            "GBps": round(nb / (ms * 1e-3) / 1e9, 1), "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "ctx": c["ctx"], "layers": c["n_layers"], "spread": round(spread, 4),
            "logits_finite": bool(np.all(np.isfinite(logits)))}


def bench_attention(iters: int, c: dict = L8B) -> dict:
    """Decode attention alone (wh_attention_decode: the partial and combine
    kernels) at the config-4 shape, position ctx - 1, over copies of the f16
    KV cache rotated so that more than 256 MB (the Infinity Cache) is in
    rotation; calls captured into a HIP graph and replayed.  Returns µs per
    call and the cache bytes read per call (2 ctx n_kv_heads head_dim 2)."""
    from woolly_amd import ops
    from woolly_amd.device import DeviceBuffer, Event, Graph, Stream

    nh, nkv, d, ctx = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ctx"]
    rng = np.random.default_rng(8)
    kc = rng.standard_normal((ctx, nkv, d)).astype(np.float16)
    vc = rng.standard_normal((ctx, nkv, d)).astype(np.float16)
    nbytes = kc.nbytes + vc.nbytes
    reps = max(1, -(-300_000_000 // nbytes))
    kbs = [DeviceBuffer.from_array(kc) for _ in range(reps)]
    vbs = [DeviceBuffer.from_array(vc) for _ in range(reps)]
    qkv = DeviceBuffer.from_array(rng.standard_normal((nh + 2 * nkv) * d).astype(np.float32))
    inv = DeviceBuffer.from_array(ops.rope_inv_freq(c["rope_base"], d))
    out = DeviceBuffer(4 * nh * d)
    wsz = ops.attention_workspace_bytes(nh, nkv, d, ctx)
    ws = DeviceBuffer(wsz)
    stream = Stream()
    pos = ctx - 1

    def run(i):
        ops.attention_decode(qkv, kbs[i % reps], vbs[i % reps], pos, nh, nkv, d, inv, out, ws, wsz, stream)

    for i in range(reps):
        run(i)
    stream.synchronize()
    ms, spread = time_graph(run, max(iters, reps), stream)
    return {"us": round(ms * 1e3, 3), "kv_bytes": nbytes, "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "ctx": ctx,
            "spread": round(spread, 4)}


def bench_host_matvec(calls: int = 20) -> dict:
    """The synchronous host-slice drop-in (quantization.simd.quantized_matvec ->
    wh_quantized_matvec_host) on the headline matrix, wall-clock µs per call
    (host arrays in, host array out, the call returns when y is on the host):
    uploading the weights on every call, and with the device copies of host
    weights on (wh_host_cache_configure), where a call after the first moves
    only x and y."""
    from woolly_amd import synth
    from woolly_amd.quantization import QuantizationScheme, QuantizedStorage, device_cache, simd

    w = synth.quantized_weight(Q4_0, N_ROWS, K, seed=3)
    x = synth.activations(K, seed=3)
    y = np.zeros(N_ROWS, np.float32)
    st = QuantizedStorage(QuantizationScheme.Q4_0, w)
    out = {}
    for name, budget in (("uploading_each_call", 0), ("cached", 1 << 30)):
        device_cache.configure(budget)
        simd.quantized_matvec(st, x, y, N_ROWS, K)  # first call (uploads when cached)
        t0 = time.perf_counter()
        for _ in range(calls):
            simd.quantized_matvec(st, x, y, N_ROWS, K)
        out[name] = round((time.perf_counter() - t0) / calls * 1e6, 1)
    device_cache.configure(0)
    return out


def bench_stream_floor(mode: int, steps: int = 200, warmup: int = 20, n: int = N_ROWS, k: int = K,
                       replicas: int = REPLICAS) -> float:
    """The read floor of the headline GEMV's access pattern (wh_read_probe): the
    same N rows of K/32 Q4_0 blocks, rotated through the same number of copies
    and timed the same way (graph replay between events, after clock settling),
    read in the GEMV's workgroup geometry without storing or computing anything.
    mode 0: one step in flight per wave, as the GEMV; mode 1: up to four;
    mode 2: not the GEMV's geometry: the same bytes as one flat range, one
    contiguous piece per workgroup, every load of a lane in flight at once.
    Returns ms per launch."""
    from woolly_amd import _lib, synth
    from woolly_amd.device import DeviceBuffer, Event, Graph, Stream

    w = synth.quantized_weight(Q4_0, n, k, seed=3)
    row_bytes = k // 32 * TYPE_SIZE[Q4_0]
    stream = Stream()
    wbufs = [DeviceBuffer.from_array(w) for _ in range(replicas)]
    out = DeviceBuffer(4 * (n // 16 + 1))  # one checksum per workgroup
    lib = _lib.load()

    def launch(i: int) -> None:
        _lib.check(lib.wh_read_probe(wbufs[i % replicas].ptr, row_bytes, n, mode, out.ptr, stream.handle))

    for i in range(warmup):
        launch(i)
    stream.synchronize()
    ms, _ = time_graph(launch, steps, stream, TIMED_LAUNCHES)
    return ms


def copy_probe(nbytes: int = 256 << 20, reps: int = 5) -> float:
    """Device-to-device copies of a known size (HIP's copy kernel): the reference
    the HBM byte counters of the GEMV are scaled by.  Returns GB/s."""
    from woolly_amd.device import DeviceBuffer, Event, Stream
    from woolly_amd import _lib

    src, dst = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    src.fill(1)
    stream = Stream()
    lib = _lib.load()
    e0, e1 = Event(), Event()
    _lib.check(lib.wh_memcpy_d2d(dst.ptr, src.ptr, nbytes, stream.handle))
    stream.synchronize()
    e0.record(stream)
    for _ in range(reps):
        _lib.check(lib.wh_memcpy_d2d(dst.ptr, src.ptr, nbytes, stream.handle))
    e1.record(stream)
    e1.synchronize()
    return 2 * nbytes * reps / (e0.elapsed_ms(e1) * 1e-3) / 1e9


# The sources each family of kernels is built from (the kernel file, the
# headers it includes).  Every summary under profiles/ names its group and
# records the digest of the group's sources: it is current only while the
# tree's sources have the same digest (checked by tests/test_bench_profile.py).
_C = "woolly_amd/csrc/"
_COMMON = (_C + "wh_common.hpp", _C + "wh_blocks.hpp")
KERNEL_SOURCE_GROUPS = {
    # single-token matrix-core GEMV and the streaming kernels it falls back to
    "gemv": (_C + "gemv_mfma.hip", _C + "gemv_mfma_dev.hpp", _C + "gemv.hip") + _COMMON,
    # several-token GEMV (2..16 tokens), one translation unit per block type
    "gemv_mt": (_C + "gemv_mt.hpp", _C + "gemv_mfma_dev.hpp", _C + "gemv_mt_q4_0.hip", _C + "gemv_mt_q4_1.hip",
                _C + "gemv_mt_q8_0.hip", _C + "gemv_mt_q4_k.hip", _C + "gemv_mt_q6_k.hip") + _COMMON,
    # tiled prefill GEMM, its packing, the K-quant conversion, the fallbacks
    "gemm": (_C + "gemm_tiled.hip", _C + "gemm.hip", _C + "kquant.hip", _C + "elementwise.hip") + _COMMON,
    "attention": (_C + "attention.hip",) + _COMMON,
}
# the decode step launches kernels of every group above and of decode.hip / embed.hip
KERNEL_SOURCE_GROUPS["decode"] = tuple(sorted(set(sum(KERNEL_SOURCE_GROUPS.values(), ())) |
                                              {_C + "decode.hip", _C + "embed.hip"}))
GEMV_KERNEL_SOURCES = KERNEL_SOURCE_GROUPS["gemv"]
PMC_PROFILE = ROOT / "profiles" / "gemv_q4_0_14336x4096_pmc.txt"


def sources_digest(paths) -> str:
    """sha256 over the given source files (paths relative to the repo root), in
    the order given, each prefixed with its path."""
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        h.update(rel.encode() + b"\0" + (ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def kernel_sources_digest(group: str = "gemv") -> str:
    """The digest of one kernel group's sources (default: the headline GEMV's)."""
    return sources_digest(KERNEL_SOURCE_GROUPS[group])


def traffic_from_profile() -> tuple[int | None, str]:
    """HBM bytes per GEMV launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE
    (scaled by the copy probe), as recorded in the committed profile summary,
    and its status: "current" when the summary's kernel_sources_sha256 matches
    the sources in this tree, else "stale" (the traffic is then reported as
    null) or "missing"."""
    fields = {}
    try:
        for line in PMC_PROFILE.read_text().splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                if v.split():
                    fields[k.strip()] = v.split()[0]  # the value, without a trailing note
    except OSError:
        return None, "missing"
    if "traffic_bytes_per_launch" not in fields:
        return None, "missing"
    if fields.get("kernel_sources_sha256") != kernel_sources_digest():
        return None, "stale"
    return int(float(fields["traffic_bytes_per_launch"])), "current"


GEMM_PMC_PROFILE = ROOT / "profiles" / "gemm_q4_0_14336x4096_m512_mfma_pmc.txt"
FP16_MFMA_PEAK_TFLOPS = 2500.0


def mfma_busy_from_profile() -> tuple[float | None, str]:
    """MFMA busy fraction of the M=512 GEMM kernel (SQ_VALU_MFMA_BUSY_CYCLES over
    all SIMD cycles) as recorded in the committed counter summary, and its
    status: "current" when the summary's kernel_sources_sha256 matches the gemm
    group's sources in this tree, else "stale" (the fraction is then null) or
    "missing"."""
    try:
        text = GEMM_PMC_PROFILE.read_text()
    except OSError:
        return None, "missing"
    digest, frac = None, None
    for line in text.splitlines():
        if line.startswith("kernel_sources_sha256:"):
            digest = line.split(":", 1)[1].split()[0]
        if line.startswith("MFMA utilisation =") and "%" in line:
            frac = float(line.split("=")[-1].split("%")[0]) / 100.0
    if frac is None:
        return None, "missing"
    if digest != kernel_sources_digest("gemm"):
        return None, "stale"
    return frac, "current"


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_calls(fn, budget_s: float) -> tuple[int, float]:
    fn()  # warm
    t0 = time.perf_counter()
    calls = 0
    while True:
        fn()
        calls += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return calls, (time.perf_counter() - t0) / calls


def cpu_baselines(budget_s: float = 8.0) -> tuple[dict | None, dict]:
    """The target GEMV on this host's CPU, timed with the test oracle:
    (1) the reference's intended SIMD path (8-lane AVX2 FMA restatement,
    nibble order fixed) on up to 16 threads -- the reported cpu_baseline;
    (2) the order-exact scalar quantized_matvec_q4_0_scalar on 1 thread, the
    reference's default x86 behaviour.  ~budget_s of CPU work each."""
    from tests._oracle import Oracle
    from woolly_amd import synth

    orc = Oracle()
    w = synth.quantized_weight(Q4_0, N_ROWS, K, seed=3)
    x = synth.activations(K, seed=3)
    nbytes = gemv_bytes(N_ROWS, K)
    cpu, nproc = _cpu_model(), os.cpu_count()
    simd = None
    if orc.simd_available():
        threads = max(1, min(16, nproc or 1))
        calls, dt = _time_calls(lambda: orc.matvec_simd_mt(Q4_0, w, x, N_ROWS, K, threads), budget_s)
        simd = {
            "value": round(nbytes / dt / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"{calls} full 14336x4096 Q4_0 GEMV calls of the oracle's restatement of "
                       f"the reference's AVX2 qmatvec_q4_0_avx2 (8-lane FMA, nibble order fixed), "
                       f"rows split over {threads} threads, {dt * 1e3:.2f} ms each, "
                       f"host '{cpu}', nproc={nproc}"),
        }
    calls, dt = _time_calls(lambda: orc.matvec_f32(Q4_0, w, x, N_ROWS, K), budget_s)
    scalar = {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{calls} full 14336x4096 Q4_0 GEMV calls of the oracle's order-exact "
                   f"quantized_matvec_q4_0_scalar restatement, {dt * 1e3:.1f} ms each, "
                   f"host '{cpu}', nproc={nproc}"),
    }
    return simd, scalar


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-ffn", action="store_true", help="skip the FFN-layer timings")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM M sweep")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other decode GEMV configurations (4096x4096 Q4_0, Q8_0, Q4_1)")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-4 decode step")
    ap.add_argument("--only", choices=["gemv", "ffn1", "ffn512", "ffn", "gemm", "decode", "decode_q4_k_m",
                                       "attention"],
                    default=None,
                    help="run one leg only (for profiling); prints that leg's timing")
    ap.add_argument("--gemm-m", type=int, default=512, help="token count of --only gemm / --only ffn")
    ap.add_argument("--type", type=int, default=Q4_0,
                    help="ggml type id of --only gemm / ffn1 / ffn512 (default Q4_0)")
    ap.add_argument("--prepared", action="store_true",
                    help="--only gemm / ffn: K-quant weights as handles converted once (wh_weight_prepare_prefill)")
    ap.add_argument("--gemv-shape", type=int, nargs=3, default=None, metavar=("TYPE", "N", "K"),
                    help="ggml type id and shape of --only gemv (default Q4_0 14336 4096)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run only device-to-device copies of 256 MiB (counter calibration)")
    ap.add_argument("--sources-digest", nargs="?", const="gemv", default=None, choices=sorted(KERNEL_SOURCE_GROUPS),
                    help="print the digest of a kernel group's sources (default: the headline GEMV's) and exit")
    args = ap.parse_args()
    if args.sources_digest:
        print(kernel_sources_digest(args.sources_digest))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path is single-GPU; it would shard by output rows, one GPU per row block)", file=sys.stderr)
        return 2

    from woolly_amd import device

    device.init(0)
    log(f"[bench] device: {device.device_name()}")
    if args.copy_probe:
        print(json.dumps({"copy_probe_GBps": round(copy_probe(), 1), "bytes_per_copy": 256 << 20}))
        return 0
    if args.only == "gemv":
        t, n, k = args.gemv_shape or (Q4_0, N_ROWS, K)
        reps = max(1, -(-300_000_000 // gemv_bytes(n, k, t)))  # > 256 MB of weights in rotation
        ms_step, _, _ = bench_gemv(args.steps, args.warmup, t, n, k, 3, reps)
        print(json.dumps({"gemv_us": round(ms_step * 1e3, 3), "type": t, "n": n, "k": k,
                          "GBps": round(gemv_bytes(n, k, t) / (ms_step * 1e-3) / 1e9, 1)}))
        return 0
    if args.only == "gemm":
        us, spread = bench_gemm(args.gemm_m, 5, args.type, prepared=args.prepared)
        print(json.dumps({f"gemm_m{args.gemm_m}_us": round(us, 2), "spread": round(spread, 4), "type": args.type,
                          "prepared": args.prepared}))
        return 0
    if args.only == "decode":
        print(json.dumps({"decode_step": bench_decode(10)}))
        return 0
    if args.only == "attention":
        print(json.dumps({"attention_decode": bench_attention(64)}))
        return 0
    if args.only == "decode_q4_k_m":
        print(json.dumps({"decode_step_q4_k_m": bench_decode(10, types=Q4_K_M, head_type=14)}))
        return 0
    if args.only in ("ffn1", "ffn512", "ffn"):
        m = 1 if args.only == "ffn1" else 512 if args.only == "ffn512" else args.gemm_m
        us, spread = bench_ffn(m, 20 if m == 1 else 3, args.type, prepared=args.prepared)
        print(json.dumps({f"ffn_m{m}_us": round(us, 2), "spread": round(spread, 4), "type": args.type,
                          "prepared": args.prepared}))
        return 0
    ms_step, med_ms, mean_ms = bench_gemv(args.steps, args.warmup)
    eager_b2b_ms, gemv_spread = bench_gemv.eager_back_to_back_ms, bench_gemv.spread
    traffic, traffic_status = traffic_from_profile()
    nbytes = gemv_bytes(N_ROWS, K)
    value = nbytes / (ms_step * 1e-3) / 1e9
    # the GEMV is the only kernel of a step: its average launch duration is the
    # timed region (graph replay, events on the launch stream) divided by K
    achieved = value
    log(f"[bench] gemv: {ms_step * 1e3:.2f} us/step in a graph (spread {gemv_spread:.3f}), eager back-to-back "
        f"{eager_b2b_ms * 1e3:.2f} us, eager between event pairs mean {mean_ms * 1e3:.2f} us (median {med_ms * 1e3:.2f})")
    # the same bytes read in the GEMV's geometry with nothing else done: what
    # this access pattern and one launch per call can reach on this part; and
    # the same bytes with every load in flight at once (the floor of one launch)
    floor = {}
    for mode, name in ((0, "gemv_geometry_1_step_in_flight"), (1, "gemv_geometry_4_steps_in_flight"),
                       (2, "flat_every_load_in_flight")):
        ms = bench_stream_floor(mode, args.steps, args.warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        floor[name] = {"us": round(ms * 1e3, 3), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"[bench] read floor ({name}): {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
    floor["gemv_us_over_floor_us"] = round(ms_step * 1e3 / floor["gemv_geometry_1_step_in_flight"]["us"], 3)
    floor["gemv_us_over_flat_floor_us"] = round(ms_step * 1e3 / floor["flat_every_load_in_flight"]["us"], 3)

    ffn, ffn_spread = {}, {}
    if not args.no_ffn:
        for m in (1, 2, 4, 512):
            us, sp = bench_ffn(m, 50 if m <= 16 else 3)
            ffn[f"m{m}"], ffn_spread[f"m{m}"] = round(us, 2), round(sp, 4)
            log(f"[bench] ffn m={m}: {ffn[f'm{m}']} us (spread {sp:.3f})"
                + (f", {us / ffn['m1']:.2f}x m=1" if m > 1 and m <= 16 else ""))

    gemm, gemm_kq = {}, {}
    if not args.no_gemm:
        # M sweep of config 2 (GEMV -> MFMA crossover).  tflops = 2*M*N*K / time;
        # the MFMA path issues two fp16 products per multiply-add (activation
        # hi and lo halves), so its MFMA work is twice that.
        for m in (1, 2, 4, 8, 16, 64, 512, 2048):
            us, sp = bench_gemm(m, 20 if m <= 64 else 5)
            tf = 2.0 * m * N_ROWS * K / (us * 1e-6) / 1e12
            gemm[f"m{m}"] = {"us": round(us, 2), "tflops": round(tf, 2), "spread": round(sp, 4)}
            log(f"[bench] gemm m={m}: {us:.2f} us, {tf:.1f} TFLOP/s (spread {sp:.3f})")
        for m in (8, 512):
            us, sp = bench_gemm(m, 20 if m <= 64 else 5, bf16=True)
            gemm[f"m{m}_bf16"] = {"us": round(us, 2), "tflops": round(2.0 * m * N_ROWS * K / (us * 1e-6) / 1e12, 2),
                                  "spread": round(sp, 4)}
            log(f"[bench] gemm bf16 activations m={m}: {us:.2f} us")
        # K-quant weights (and Q4_1): a few tokens stream the blocks once
        # (several-token GEMV); at M=512 the tiled GEMM, on a copy converted
        # once per handle (wh_weight_prepare_prefill) and, for comparison, with
        # the conversion inside every call
        for name, t in (("q4_k", 12), ("q6_k", 14), ("q4_1", 3)):
            for m in ((1, 2, 8, 16) if t == 12 else (1, 8)):
                us, sp = bench_gemm(m, 20, t)
                gemm_kq[f"gemm_{name}_m{m}"] = {"us": round(us, 2), "spread": round(sp, 4)}
                log(f"[bench] gemm {name} m={m}: {us:.2f} us")
            if t == 3:  # no conversion: the tiled GEMM reads Q4_1 blocks as they are
                us, sp = bench_gemm(512, 5, t)
                tf = 2.0 * 512 * N_ROWS * K / (us * 1e-6) / 1e12
                gemm_kq["gemm_q4_1_m512"] = {"us": round(us, 2), "tflops": round(tf, 2), "spread": round(sp, 4)}
                log(f"[bench] gemm q4_1 m=512: {us:.2f} us, {tf:.1f} TFLOP/s")
                continue
            for prep in (True, False):
                us, sp = bench_gemm(512, 5, t, prepared=prep)
                tf = 2.0 * 512 * N_ROWS * K / (us * 1e-6) / 1e12
                key = f"gemm_{name}_m512" + ("" if prep else "_converting")
                gemm_kq[key] = {"us": round(us, 2), "tflops": round(tf, 2), "spread": round(sp, 4)}
                log(f"[bench] gemm {name} m=512{'' if prep else ' (conversion per call)'}: {us:.2f} us, "
                    f"{tf:.1f} TFLOP/s")
        if not args.no_ffn:
            for name, t in (("q4_k", 12), ("q6_k", 14)):
                us1, _ = bench_ffn(1, 50, t)
                us512, sp = bench_ffn(512, 3, t, prepared=True)
                gemm_kq[f"ffn_{name}_m1_us"] = round(us1, 2)
                gemm_kq[f"ffn_{name}_m512_us"] = round(us512, 2)
                log(f"[bench] ffn {name}: m=1 {us1:.2f} us, m=512 {us512:.2f} us (prepared handles)")
            us512, _ = bench_ffn(512, 3, 3)
            gemm_kq["ffn_q4_1_m512_us"] = round(us512, 2)
            log(f"[bench] ffn q4_1: m=512 {us512:.2f} us")

    # the other decode GEMV configurations (config 0, 1a, 1b); replicas keep
    # each timed set of weights above the 256 MB Infinity Cache
    gemv_cfg = {}
    if not args.no_configs:
        for name, t, n, k, seed, reps in (("c0_q4_0_4096x4096", Q4_0, 4096, 4096, 0, 32),
                                          ("c1a_q8_0_14336x4096", 8, 14336, 4096, 1, 5),
                                          ("c1b_q4_1_14336x4096", 3, 14336, 4096, 2, 8),
                                          # decode-step shapes: k/v projections, FFN down,
                                          # the Q8_0 output head
                                          ("attn_kv_q4_0_1024x4096", Q4_0, 1024, 4096, 6, 120),
                                          ("ffn_down_q4_0_4096x14336", Q4_0, 4096, 14336, 6, 10),
                                          ("head_q8_0_128256x4096", 8, 128256, 4096, 6, 1),
                                          # the K-quant blocks (woolly-gguf's Q4_K / Q6_K layout)
                                          ("kq_q4_k_14336x4096", 12, 14336, 4096, 7, 10),
                                          ("kq_q6_k_14336x4096", 14, 14336, 4096, 7, 7),
                                          ("kq_q4_k_4096x14336", 12, 4096, 14336, 7, 10),
                                          ("kq_q6_k_4096x14336", 14, 4096, 14336, 7, 7)):
            ms, _, _ = bench_gemv(100, 10, t, n, k, seed, reps)
            gbs = gemv_bytes(n, k, t) / (ms * 1e-3) / 1e9
            gemv_cfg[name] = {"us": round(ms * 1e3, 3), "GBps": round(gbs, 1),
                              "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": gemv_bytes(n, k, t),
                              "spread": round(bench_gemv.spread, 4)}
            log(f"[bench] gemv {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")

    host_mv = None
    if not args.no_configs:
        host_mv = bench_host_matvec()
        log(f"[bench] host-slice GEMV (wh_quantized_matvec_host), us per call: {host_mv}")

    decode = decode_km = attn = None
    if not args.no_decode:
        attn = bench_attention(64)
        log(f"[bench] decode attention (config 4 shape, ctx {attn['ctx']}): {attn['us']} us, {attn['GBps']} GB/s "
            f"over the {attn['kv_bytes']} cache bytes")
        decode = bench_decode(20)
        log(f"[bench] decode step (config 4, ctx {decode['ctx']}): {decode['ms_per_token']} ms/token, "
            f"{decode['tokens_per_s']} tokens/s, {decode['GBps']} GB/s")
        decode_km = bench_decode(10, types=Q4_K_M, head_type=14)
        log(f"[bench] decode step Q4_K_M types (ctx {decode_km['ctx']}): {decode_km['ms_per_token']} ms/token, "
            f"{decode_km['tokens_per_s']} tokens/s, {decode_km['GBps']} GB/s")

    cpu, cpu_scalar = (None, None) if args.no_cpu else cpu_baselines()
    if cpu:
        log(f"[bench] cpu baseline (simd, {cpu['cores']} threads): {cpu['value']} GB/s")
    if cpu_scalar:
        log(f"[bench] cpu baseline (scalar, 1 thread): {cpu_scalar['value']} GB/s")

    # MFMA utilisation of the M=512 GEMM: issued fp16 MFMA work (the activation
    # hi and lo halves, 2 x 2 M N K) over the call's time against the dense
    # peak, and the counters' busy fraction of the kernel from the committed
    # summary of the same sources
    prefill_mfma = None
    if gemm.get("m512"):
        busy, busy_status = mfma_busy_from_profile()
        issued = 2.0 * 2.0 * 512 * N_ROWS * K / (gemm["m512"]["us"] * 1e-6) / 1e12
        prefill_mfma = {"issued_tflops": round(issued, 1), "peak_tflops": FP16_MFMA_PEAK_TFLOPS,
                        "issued_frac_of_peak": round(issued / FP16_MFMA_PEAK_TFLOPS, 4),
                        "counters_busy_frac": round(busy, 4) if busy is not None else None,
                        "counters_profile": f"{GEMM_PMC_PROFILE.relative_to(ROOT)} ({busy_status})"}
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64: d=f16(|N(0,0.02)|), uniform nibbles, x~N(0,1))",
        "config": {
            "workload": "Q4_0 decode GEMV N=14336 x K=4096 (FFN gate/up), f32 x and y, "
                        f"{REPLICAS} rotating weight copies in HBM",
            "n_rows": N_ROWS, "k": K, "ggml_type": "Q4_0", "bytes_per_launch": nbytes,
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_profile": f"{PMC_PROFILE.relative_to(ROOT)} ({traffic_status})",
            "kernel": "gemv_mfma_kernel<Q4_0, 1 K-segment, 3 loads/step, plain> (int8 MFMA)",
            "profile": "profiles/gemv_q4_0_14336x4096_kernel_trace.txt",
            "launch_us_mean": round(ms_step * 1e3, 3),
            "launches_timed": bench_gemv.launches_timed,
            "launch_us_eager_event_pairs": round(mean_ms * 1e3, 3),
            "launch_us_eager_back_to_back": round(eager_b2b_ms * 1e3, 3),
            "spread": round(gemv_spread, 4),
            "read_floor": floor,
        },
        "ffn_layer_us": ffn or None,
        "ffn_layer_spread": ffn_spread or None,
        "prefill_gemm_q4_0_14336x4096": gemm or None,
        "prefill_mfma_m512": prefill_mfma,
        "prefill_kquant_14336x4096": gemm_kq or None,
        "gemv_other_configs": gemv_cfg or None,
        "host_slice_gemv_q4_0_14336x4096_us": host_mv,
        "decode_step_llama3_8b_q4_0": decode,
        "decode_step_llama3_8b_q4_k_m": decode_km,
        "decode_attention_llama3_8b_ctx4096": attn,
        "cpu_baseline": cpu,
        "cpu_baseline_scalar": cpu_scalar,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
