"""Benchmark of the quantized-weight path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu]

Headline (one JSON line on stdout): MatMulNBits q4 decode GEMV throughput in GB/s at M=1 on
the Qwen3-0.6B projection shapes (block 32, f16 activations and scales, packed zero points).
One step is one decode step's 196 projection GEMVs (28 layers x q, k, v, o, gate, up, down),
each layer with its own weights; consecutive steps rotate over 4 copies of the 28 layers
(1.02 GB of packed weights, 4x the 256 MB last-level cache) so the bytes come from HBM.
Each step is one HIP graph of 196 launches on the library's stream; the timed region is K
replays between two HIP events. GB/s counts the algorithmic bytes of each call: packed
weights + scales + packed zero points + A + Y.

The same line carries the M = 4/8/16 decode sweep, the prefill GEMM at SmolLM3-3B shapes
(M = 256 and 2048, block 128, TFLOP/s), the large-vocabulary GatherBlockQuantized and lm_head,
the roofline of the dominant kernel, and a CPU baseline: the reference's EXLA-CPU path after
move/2 (weights dequantized once to f16, then an f32-accumulating GEMV on host threads),
restated in C (oracle/oracle.c) and timed on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA

# Qwen3-0.6B decode projections: (name, K, N)
QWEN3_06B = [("q", 1024, 2048), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 2048, 1024),
             ("gate", 1024, 3072), ("up", 1024, 3072), ("down", 3072, 1024)]
QWEN3_LAYERS = 28
# SmolLM3-3B prefill projections: (name, K, N)
SMOLLM3_3B = [("attn 2048->2048", 2048, 2048), ("mlp 2048->11008", 2048, 11008), ("mlp 11008->2048", 11008, 2048)]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def nbits_bytes(k, n, m, bits=4, bs=32, scale_bytes=2, zp=True, a_bytes=2, y_bytes=2):
    """Algorithmic bytes of one MatMulNBits call."""
    blocks = -(-k // bs)
    total = n * blocks * bs * bits // 8 + n * blocks * scale_bytes
    if zp:
        total += n * (-(-blocks * bits // 8))
    return total + m * k * a_bytes + m * n * y_bytes


def make_weight_parts(rng, k, n, bits=4, bs=32, scale_mul=0.01):
    blocks = -(-k // bs)
    b = rng.integers(0, 256, (n, blocks, bs * bits // 8), dtype=np.uint8)
    scales = (np.abs(rng.standard_normal(n * blocks, dtype=np.float32)) * scale_mul + 1e-4).astype(np.float16)
    zp = rng.integers(0, 256, n * (-(-blocks * bits // 8)), dtype=np.uint8)
    return b, scales, zp


class Timer:
    """HIP events on the library's stream."""

    def __init__(self, ctx):
        from transmuter_amd._lib import lib

        self.ctx, self.lib = ctx, lib()
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        ctx.check(self.lib.tmh_event_create(ctx.handle, ctypes.byref(self.a)))
        ctx.check(self.lib.tmh_event_create(ctx.handle, ctypes.byref(self.b)))

    def start(self):
        self.ctx.check(self.lib.tmh_event_record(self.ctx.handle, self.a, None))

    def stop_ms(self) -> float:
        self.ctx.check(self.lib.tmh_event_record(self.ctx.handle, self.b, None))
        ms = ctypes.c_float()
        self.ctx.check(self.lib.tmh_event_elapsed(self.ctx.handle, self.a, self.b, ctypes.byref(ms)))
        return ms.value


class Graph:
    """A HIP graph recorded from calls on the library's stream. With USE_GRAPHS off (the
    --no-graph flag, for tracers that do not follow graph launches) the calls are replayed
    directly on the stream instead."""

    def __init__(self, ctx, record):
        from transmuter_amd._lib import lib

        self.ctx, self.lib, self.record = ctx, lib(), record
        self.exec = None
        if not USE_GRAPHS:
            return
        ctx.check(self.lib.tmh_graph_begin(ctx.handle, None))
        try:
            record()
        finally:
            self.exec = ctypes.c_void_p()
            ctx.check(self.lib.tmh_graph_end(ctx.handle, None, ctypes.byref(self.exec)))

    def launch(self):
        if self.exec is None:
            self.record()
        else:
            self.ctx.check(self.lib.tmh_graph_launch(self.ctx.handle, self.exec, None))

    def destroy(self):
        if self.exec is not None:
            self.ctx.check(self.lib.tmh_graph_destroy(self.ctx.handle, self.exec))


USE_GRAPHS = True
STAMP_HEADLINE = True  # time the headline's kernels inside the replays too (--no-timeline turns it off)


def rocprof_domains() -> list[str]:
    """The rocprofv3 tracing or counter-collection domains switched on in this process's
    environment (rocprofv3 exports ROCPROF_<DOMAIN>_TRACE=1 and ROCPROF_COUNTER_COLLECTION=1)."""
    return sorted(k for k, v in os.environ.items()
                  if k.startswith("ROCPROF_") and (k.endswith("_TRACE") or k == "ROCPROF_COUNTER_COLLECTION")
                  and v == "1")


# Graph replays under rocprofv3 ended twice in a segmentation fault inside hipGraphLaunch, at the
# same code offset of the runtime, once in a process that never loaded this library: the tracer's
# own graph-launch path. Runs under the tracer therefore launch every call directly (--profile,
# --no-graph); a graph run under it is refused.
GRAPHS_UNDER_TRACER = "graph replays are not run under rocprofv3 (its graph-launch path has crashed)"


def matmul_call(ctx, w, a, y, m):
    from transmuter_amd._lib import lib

    ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, a.tmh_dtype, m, w.k, None, 0, y.ptr, y.tmh_dtype, w.n,
                                     None))


def time_graphs(ctx, graphs, steps, warmup):
    for i in range(warmup):
        graphs[i % len(graphs)].launch()
    ctx.synchronize()
    t = Timer(ctx)
    t.start()
    for i in range(steps):
        graphs[i % len(graphs)].launch()
    return t.stop_ms()


# ---------------------------------------------------------------- decode sweep (headline)


def decode_sweep(ctx, steps, warmup, sets, ms, merged=False, full_step=False):
    """merged: q/k/v and gate/up run as one call each over concatenated weights, as the
    reference's move/2 + Fusion.matmuls/2 leave a Qwen3 layer (4 calls instead of 7).
    full_step: also time a whole decode step, the 196 layer GEMVs and the 151936 x 1024
    lm_head in one graph, and the host-observed latency of one eagerly launched 1024 -> 3072
    GEMV (launch and synchronize); at M=1 also the floors (an empty kernel per projection, a
    plain read of each projection's packed weights) and the step launched eagerly."""
    from transmuter_amd import PackedWeight

    rng = np.random.default_rng(20260101)
    log(f"decode: packing {sets} x {QWEN3_LAYERS} layers of Qwen3-0.6B q4 weights")
    t0 = time.time()
    weights = []  # weights[s][layer][proj]
    for s in range(sets):
        layer_ws = []
        for _layer in range(QWEN3_LAYERS):
            row = []
            for _name, k, n in QWEN3_06B:
                b, sc, zp = make_weight_parts(rng, k, n)
                row.append(PackedWeight.upload(ctx, b, sc, zp, k=k, n=n, bits=4, block_size=32, weight_dtype="f16"))
            layer_ws.append(row)
        if merged:
            layer_ws = [[PackedWeight.concat(row[0:3]), row[3], PackedWeight.concat(row[4:6]), row[6]]
                        for row in layer_ws]
        weights.append(layer_ws)
    log(f"decode: packed {sum(w.device_bytes() for ls in weights for l in ls for w in l) / 1e9:.2f} GB "
        f"in {time.time() - t0:.1f} s")
    results = {}
    for m in ms:
        a = {k: ctx.put(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)) for k in (1024, 2048, 3072)}
        y = {n: ctx.empty((m, n), "f16") for n in (1024, 2048, 3072)}
        for n in (4096, 6144):
            y[n] = ctx.empty((m, n), "f16")
        graphs = []
        for s in range(sets):
            def record(s=s):
                for layer in range(QWEN3_LAYERS):
                    for w in weights[s][layer]:
                        matmul_call(ctx, w, a[w.k], y[w.n], m)
            graphs.append(Graph(ctx, record))
        step_bytes = QWEN3_LAYERS * sum(nbits_bytes(w.k, w.n, m) for w in weights[0][0])
        step_flops = QWEN3_LAYERS * sum(2 * m * k * n for _name, k, n in QWEN3_06B)
        ms_total = time_graphs(ctx, graphs, steps, warmup)
        ms_step = ms_total / steps
        per_layer = len(weights[0][0])
        launches = steps * QWEN3_LAYERS * per_layer
        results[m] = {
            "M": m, "gbs": step_bytes / (ms_step * 1e-3) / 1e9, "ms_per_step": ms_step,
            "tflops": step_flops / (ms_step * 1e-3) / 1e12, "tokens_per_s": m * 1e3 / ms_step,
            "us_per_launch": ms_total * 1e3 / launches, "bytes_per_launch": step_bytes / (QWEN3_LAYERS * per_layer),
            "step_bytes": step_bytes,
        }
        log(f"decode{' merged' if merged else ''} M={m}: {ms_step * 1e3:.1f} us/step, {results[m]['gbs']:.0f} GB/s, "
            f"{results[m]['us_per_launch']:.2f} us/launch")
        for g in graphs:
            g.destroy()
        if full_step and m == 1 and not merged and STAMP_HEADLINE and USE_GRAPHS:
            # The same step's kernels timed inside the replays (launch timeline), two rotations.
            calls = [(f"{name} {k}->{n}", nbits_bytes(k, n, m), 2 * m * k * n) for _layer in range(QWEN3_LAYERS)
                     for name, k, n in QWEN3_06B]
            res = timeline_steps(ctx, [lambda s=s: [matmul_call(ctx, w, a[w.k], y[w.n], m)
                                                    for layer in weights[s % sets] for w in layer]
                                       for s in range(2 * sets)], calls, reps=steps, warmup=warmup)
            results[m]["timeline"] = timeline_summary(res)
        if (full_step or merged) and m == 1:
            results[m].update(decode_floors(ctx, steps, warmup, weights, lambda s: [
                matmul_call(ctx, w, a[w.k], y[w.n], m) for layer in range(QWEN3_LAYERS) for w in weights[s][layer]],
                label="decode merged floors" if merged else "decode floors"))
        if full_step:
            results[m].update(full_decode_step(ctx, steps, warmup, weights, a, y, m))
    for ls in weights:
        for layer in ls:
            for w in layer:
                w.free()
    return results


def decode_floors(ctx, steps, warmup, weights, eager_step, label="decode floors"):
    """What one launch per projection costs without the GEMV's work, in graphs of the same
    launches (196 per step, 112 with q/k/v and gate/up merged) rotating over the same weight
    copies: an empty kernel (the launch floor) and a plain read of each projection's packed
    weights with the GEMV's load pattern (the read floor). Also the decode step's GEMVs launched
    eagerly, back to back, with one synchronize at the end."""
    from transmuter_amd._lib import lib

    per_step = QWEN3_LAYERS * len(weights[0][0])
    empty = [Graph(ctx, lambda: [ctx.check(lib().tmh_floor_empty(ctx.handle, 256, None)) for _ in range(per_step)])]
    launch_us = time_graphs(ctx, empty, steps, warmup) * 1e3 / (steps * per_step)
    empty[0].destroy()
    sink = ctx.empty((16,), "u8")
    reads = [Graph(ctx, lambda s=s: [ctx.check(lib().tmh_floor_read(ctx.handle, w.handle, sink.ptr, None))
                                     for layer in range(QWEN3_LAYERS) for w in weights[s][layer]])
             for s in range(len(weights))]
    read_us = time_graphs(ctx, reads, steps, warmup) * 1e3 / (steps * per_step)
    for g in reads:
        g.destroy()
    q_bytes = QWEN3_LAYERS * sum(-(-w.n // 16) * -(-(w.k * w.bits // 8) // 64) * 1024 for w in weights[0][0])
    for i in range(warmup):
        eager_step(i % len(weights))
    ctx.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        eager_step(i % len(weights))
    ctx.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    log(f"{label}: empty kernel {launch_us:.2f} us/launch, plain read of the packed weights {read_us:.2f} "
        f"us/launch ({q_bytes / (read_us * per_step * 1e-6) / 1e9:.0f} GB/s); eager step {eager_ms * 1e3:.0f} us "
        f"({1e3 / eager_ms:.0f} tokens/s)")
    return {"launch_floor_us": launch_us, "read_floor_us": read_us,
            "read_floor_gbs": q_bytes / (read_us * per_step * 1e-6) / 1e9,
            "eager_ms_per_step": eager_ms, "eager_tokens_per_s": 1e3 / eager_ms}


def full_decode_step(ctx, steps, warmup, weights, a, y, m, vocab=151936, hidden=1024):
    """A whole synthetic Qwen3-0.6B decode step (28 layers of 7 GEMVs, then the lm_head over
    the tied 151936 x 1024 embedding) per graph, rotating over the layer weight copies, and the
    host-observed latency of one eager 1024 -> 3072 GEMV."""
    from transmuter_amd import PackedWeight

    rng = np.random.default_rng(7)
    b, sc, zp = make_weight_parts(rng, hidden, vocab)
    lm = PackedWeight.upload(ctx, b, sc, zp, k=hidden, n=vocab, bits=4, block_size=32, weight_dtype="f16")
    y_lm = ctx.empty((m, vocab), "f16")
    graphs = []
    for s in range(len(weights)):
        def record(s=s):
            for layer in range(QWEN3_LAYERS):
                for w in weights[s][layer]:
                    matmul_call(ctx, w, a[w.k], y[w.n], m)
            matmul_call(ctx, lm, a[hidden], y_lm, m)
        graphs.append(Graph(ctx, record))
    ms_step = time_graphs(ctx, graphs, steps, warmup) / steps
    for g in graphs:
        g.destroy()
    gate = weights[0][0][4]
    for _ in range(20):
        matmul_call(ctx, gate, a[gate.k], y[gate.n], m)
        ctx.synchronize()
    reps = 200
    t0 = time.perf_counter()
    for _ in range(reps):
        matmul_call(ctx, gate, a[gate.k], y[gate.n], m)
        ctx.synchronize()
    single_us = (time.perf_counter() - t0) * 1e6 / reps
    lm.free()
    log(f"decode step with lm_head M={m}: {ms_step * 1e3:.1f} us/step, {m * 1e3 / ms_step:.0f} tokens/s; "
        f"one eager 1024->3072 GEMV, launch to synchronize: {single_us:.1f} us")
    return {"ms_per_step_with_lm_head": ms_step, "tokens_per_s_with_lm_head": m * 1e3 / ms_step,
            "single_launch_us": single_us}


# ---------------------------------------------------------------- single op (the CPU-path config)


def single_op(ctx, reps, copies=160):
    """The single MatMulNBits op of the reference's EXLA-CPU configuration: A f32 [1, 1024],
    B [3072, 32, 16] of uniform nibbles, f32 scales |N(0,1)|*0.01+1e-4, no zero points, Y f32
    [1, 3072]. Weights dequantize in the scales' type (f32), as move/2 leaves them. One graph of
    `copies` calls over distinct weight copies (304 MB, more than the 256 MB last-level cache)."""
    from transmuter_amd import PackedWeight
    from transmuter_amd._lib import F32, lib

    rng = np.random.default_rng(1)
    k, n = 1024, 3072
    ws = []
    for _ in range(copies):
        b = rng.integers(0, 256, (n, k // 32, 16), dtype=np.uint8)
        sc = (np.abs(rng.standard_normal(n * k // 32, dtype=np.float32)) * 0.01 + 1e-4).astype(np.float32)
        ws.append(PackedWeight.upload(ctx, b, sc, None, k=k, n=n, bits=4, block_size=32, weight_dtype="f32"))
    a = ctx.put(rng.standard_normal((1, k), dtype=np.float32))
    y = ctx.empty((1, n), "f32")
    g = Graph(ctx, lambda: [ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, F32, 1, k, None, 0, y.ptr,
                                                             F32, n, None)) for w in ws])
    us = time_graphs(ctx, [g], reps, 2) * 1e3 / (reps * copies)
    g.destroy()
    for w in ws:
        w.free()
    nbytes = nbits_bytes(k, n, 1, scale_bytes=4, zp=False, a_bytes=4, y_bytes=4)
    log(f"single op K=1024 N=3072 f32: {us:.2f} us, {nbytes / us / 1e3:.0f} GB/s")
    return {"us": us, "gbs": nbytes / (us * 1e-6) / 1e9}


# ---------------------------------------------------------------- prefill GEMM


NP_TYPES = {"f16": np.float16, "f32": np.float32}
ROTATE_BYTES = 1 << 30  # weight copies a workload's calls rotate over: 4x the 256 MB last-level cache


def prefill(ctx, reps, ms_list, per_graph=8, rotate_bytes=ROTATE_BYTES, dtype="f16"):
    """SmolLM3-3B projections, q4 block 128, at each M: `per_graph` calls per graph. Each
    projection's calls rotate over device copies of its weight totalling `rotate_bytes` (four
    times the 256 MB last-level cache), so the weights stream from HBM as a model's would; the
    graphs are replayed round robin, each at least once per timed run. `dtype` is the type of A,
    of the weights (their scales converted to it) and of Y: f16, bf16 or f32."""
    from transmuter_amd import PackedWeight
    from transmuter_amd.device import f32_to_bf16_bits

    rng = np.random.default_rng(3)
    out = {}
    ws = []
    for _name, k, n in SMOLLM3_3B:
        b, sc, zp = make_weight_parts(rng, k, n, bs=128, scale_mul=0.005)
        w = PackedWeight.upload(ctx, b, sc, zp, k=k, n=n, bits=4, block_size=128, weight_dtype=dtype)
        copies = max(1, -(-rotate_bytes // w.device_bytes()))
        copies = -(-copies // per_graph) * per_graph
        ws.append([w] + [PackedWeight.concat([w]) for _ in range(copies - 1)])
    for m in ms_list:
        per = []
        for (name, k, n), copies in zip(SMOLLM3_3B, ws):
            a32 = rng.standard_normal((m, k), dtype=np.float32)
            a = ctx.put(f32_to_bf16_bits(a32), "bf16") if dtype == "bf16" else ctx.put(a32.astype(NP_TYPES[dtype]))
            y = ctx.empty((m, n), dtype)
            matmul_call(ctx, copies[0], a, y, m)  # eager first: sizes the split-K workspace before capture
            ctx.synchronize()
            graphs = [Graph(ctx, lambda i=i, a=a, y=y: [matmul_call(ctx, copies[i + j], a, y, m) for j in range(per_graph)])
                      for i in range(0, len(copies), per_graph)]
            steps = max(reps, len(graphs))
            ms_total = time_graphs(ctx, graphs, steps, 3)
            for g in graphs:
                g.destroy()
            us = ms_total * 1e3 / (steps * per_graph)
            flops = 2 * m * k * n
            per.append({"proj": name, "M": m, "us": us, "tflops": flops / (us * 1e-6) / 1e12,
                        "weight_copies": len(copies)})
            log(f"prefill {dtype} {name} M={m}: {us:.1f} us, {per[-1]['tflops']:.1f} TFLOP/s ({len(copies)} weight copies)")
            a.free()
            y.free()
        flops = sum(2 * m * k * n for _name, k, n in SMOLLM3_3B)
        us = sum(p["us"] for p in per)
        out[m] = {"tflops": flops / (us * 1e-6) / 1e12, "per_projection": per}
    for copies in ws:
        for w in copies:
            w.free()
    return out


# ---------------------------------------------------------------- large vocabulary


def large_vocab(ctx, reps, per_graph=21):
    """lm_head MatMulNBits (M=1 and M=8) and the tied-embedding GatherBlockQuantized lookup. Each
    graph holds `per_graph` calls, so one graph launch's own cost spreads over them; the lm_head
    calls rotate over 12 weight copies (1.1 GB, four times the 256 MB last-level cache) and
    every gather call reads its own 4096 ids, from 2 tables."""
    from transmuter_amd import PackedWeight
    from transmuter_amd._lib import F16, S64, U8, lib

    rng = np.random.default_rng(4)
    vocab, hidden = 151936, 1024
    b, sc, zp = make_weight_parts(rng, hidden, vocab)
    ws = [PackedWeight.upload(ctx, b, sc, zp, k=hidden, n=vocab, bits=4, block_size=32, weight_dtype="f16")]
    ws += [PackedWeight.concat([ws[0]]) for _ in range(-(-ROTATE_BYTES // ws[0].device_bytes()) - 1)]
    out = {}
    for m in (1, 8):
        a = ctx.put(rng.standard_normal((m, hidden), dtype=np.float32).astype(np.float16))
        y = ctx.empty((m, vocab), "f16")

        def lm_heads(a=a, y=y, m=m):
            for i in range(per_graph):
                matmul_call(ctx, ws[i % len(ws)], a, y, m)

        g = Graph(ctx, lm_heads)
        us = time_graphs(ctx, [g], reps, 3) * 1e3 / (reps * per_graph)
        g.destroy()
        lm_bytes = nbits_bytes(hidden, vocab, m)
        out[f"lm_head_M{m}"] = {"us": us, "gbs": lm_bytes / (us * 1e-6) / 1e9,
                                "frac": lm_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        log(f"lm_head M={m}: {us:.1f} us, {lm_bytes / us / 1e3:.0f} GB/s")
    # The read floor at this shape: a plain read of each copy's packed weights (the GEMV's load
    # pattern, not its scales and zero points) over the same rotation.
    sink = ctx.empty((16,), "u8")
    g = Graph(ctx, lambda: [ctx.check(lib().tmh_floor_read(ctx.handle, ws[i % len(ws)].handle, sink.ptr, None))
                            for i in range(per_graph)])
    us = time_graphs(ctx, [g], reps, 3) * 1e3 / (reps * per_graph)
    g.destroy()
    q_bytes = vocab * hidden // 2
    out["lm_head_read_floor"] = {"us": us, "gbs": q_bytes / (us * 1e-6) / 1e9, "weight_copies": len(ws)}
    log(f"lm_head read floor: {us:.1f} us for the {q_bytes / 1e6:.1f} MB of packed weights, "
        f"{q_bytes / us / 1e3:.0f} GB/s ({len(ws)} copies)")
    for w in ws:
        w.free()
    tables = [(ctx.put(b.reshape(vocab, -1)), ctx.put(sc.reshape(vocab, -1)), ctx.put(zp.reshape(vocab, -1)))
              for _ in range(2)]
    ids = [ctx.put(rng.integers(0, vocab, (8, 512)).astype(np.int64)) for _ in range(per_graph)]
    rows = ctx.empty((8, 512, hidden), "f16")

    def gathers():
        for i in range(per_graph):
            table, scales, zps = tables[i % 2]
            ctx.check(lib().tmh_gather_block_quantized(ctx.handle, table.ptr, U8, vocab, hidden // 2, ids[i].ptr, S64,
                                                       4096, scales.ptr, F16, hidden // 32, zps.ptr, U8, 4, rows.ptr,
                                                       None))

    g2 = Graph(ctx, gathers)
    us_g = time_graphs(ctx, [g2], reps, 3) * 1e3 / (reps * per_graph)
    g2.destroy()
    g_bytes = 4096 * (hidden // 2 + hidden // 32 * 2 + hidden // 64 + 8) + 4096 * hidden * 2
    log(f"gather: {us_g:.1f} us, {g_bytes / us_g / 1e3:.0f} GB/s")
    out["gather_8x512"] = {"us": us_g, "gbs": g_bytes / (us_g * 1e-6) / 1e9}
    return out


# ---------------------------------------------------------------- quantized MoE


def moe_ffn(ctx, reps, per_graph=6, sets=3):
    """QMoE at the Qwen3-30B-A3B expert shape: 128 experts, top-8 routing, hidden 2048,
    intermediate 768, SwiGLU (gate fc1, linear fc3, down fc2), q4 block 32 with f16 scales (no
    zero points), 512 tokens of f16 activations and N(0,1) router logits; routing, grouping, the
    three grouped expert products, activation and the weighted sum in each call. The calls
    rotate over `sets` device copies of the layer's expert weights (3: 1.05 GB, four times the
    256 MB last-level cache)."""
    import ctypes

    from transmuter_amd._lib import F16, F32, lib
    from transmuter_amd.moe import ExpertWeight

    rng = np.random.default_rng(6)
    experts, k, hidden, inter, tokens = 128, 8, 2048, 768, 512

    def expert_weight(n, kk):
        packed = rng.integers(0, 256, (experts, n, kk // 2), dtype=np.uint8)
        scales = (np.abs(rng.standard_normal((experts, n, kk // 32), dtype=np.float32)) * 0.01 + 1e-4).astype(np.float16)
        return ExpertWeight.upload(ctx, packed, scales, None, bits=4, block_size=32, dtype="f16")

    def device_copy(w):
        handle = ctypes.c_void_p()
        ctx.check(lib().tmh_weight_concat_nbits(ctx.handle, (ctypes.c_void_p * 1)(w.handle.value), 1,
                                                ctypes.byref(handle)))
        return ExpertWeight(ctx, handle, w.experts, w.n, w.k, w.bits, w.dtype)

    first = (expert_weight(inter, hidden), expert_weight(inter, hidden), expert_weight(hidden, inter))
    layers = [first] + [tuple(device_copy(w) for w in first) for _ in range(sets - 1)]
    x = ctx.put(rng.standard_normal((tokens, hidden), dtype=np.float32).astype(np.float16))
    router = ctx.put(rng.standard_normal((tokens, experts), dtype=np.float32))
    y = ctx.empty((tokens, hidden), "f16")

    def call(i):
        fc1, fc3, fc2 = layers[i % len(layers)]
        ctx.check(lib().tmh_qmoe(ctx.handle, x.ptr, F16, tokens, hidden, router.ptr, F32, experts, k, fc1.handle, None,
                                 fc2.handle, None, fc3.handle, None, F16, 4, 0, 1.0, 0.0, 0.0, y.ptr, None))

    call(0)  # eager first: sizes the workspace before capture
    ctx.synchronize()
    g = Graph(ctx, lambda: [call(i) for i in range(per_graph)])
    us = time_graphs(ctx, [g], reps, 2) * 1e3 / (reps * per_graph)
    g.destroy()
    for layer in layers:
        for w in layer:
            w.free()
    flops = tokens * k * 2 * 3 * hidden * inter
    weight_bytes = experts * 3 * hidden * inter * (0.5 + 2 / 32)
    log(f"moe 128x top-8 2048/768 T={tokens}: {us:.1f} us, {flops / us / 1e6:.1f} TFLOP/s, "
        f"{tokens / us * 1e6:.0f} tokens/s, {weight_bytes / us / 1e3:.0f} GB/s of expert weights")
    return {"us": us, "tflops": flops / (us * 1e-6) / 1e12, "tokens_per_s": tokens / (us * 1e-6),
            "weight_gbs": weight_bytes / (us * 1e-6) / 1e9}


# ---------------------------------------------------------------- 8-bit integer path


def int8_ops(ctx, reps, per_graph=8, m=2048, k=2048, n=2048):
    """The dynamic-quantization path at a 2048 x 2048 x 2048 projection: DynamicQuantizeLinear of
    f32 activations, MatMulInteger of u8 activations (one zero point) with u8 weights (a zero
    point per column) into s32 on the int8 MFMA, and a per-axis DequantizeLinear of u8 [2048,
    2048] to f32. `per_graph` calls per HIP graph."""
    from transmuter_amd._lib import F32, U8, QPARAM_AXIS, lib

    rng = np.random.default_rng(7)
    x = ctx.put(rng.standard_normal((m, k), dtype=np.float32))
    xq, xs, xz = ctx.empty((m, k), "u8"), ctx.empty((), "f32"), ctx.empty((), "u8")
    bq = ctx.put(rng.integers(0, 256, (k, n), dtype=np.uint8))
    bz = ctx.put(rng.integers(0, 256, n, dtype=np.uint8))
    y = ctx.empty((m, n), "s32")
    scale = ctx.put((np.abs(rng.standard_normal(k)) * 0.01 + 1e-3).astype(np.float32))
    dq = ctx.empty((m, k), "f32")

    def dql():
        ctx.check(lib().tmh_dynamic_quantize_linear(ctx.handle, x.ptr, F32, m * k, xq.ptr, xs.ptr, xz.ptr, None))

    def mmi():
        ctx.check(lib().tmh_matmul_integer(ctx.handle, xq.ptr, U8, bq.ptr, U8, xz.ptr, 1, bz.ptr, n, 1, m, k, n, 0,
                                           y.ptr, None))

    def dl():
        ctx.check(lib().tmh_dequantize_linear(ctx.handle, xq.ptr, U8, m, k, 1, scale.ptr, F32, None, 0, QPARAM_AXIS,
                                              0, dq.ptr, None))

    from transmuter_amd.packed import Int8Weight

    bw = Int8Weight.prepare(ctx, bq, bz)  # the weight initializer as the load-time move prepares it

    def mmi_prepared():
        ctx.check(lib().tmh_matmul_integer_prepared(ctx.handle, xq.ptr, U8, xz.ptr, 1, 1, m, bw.handle, y.ptr, None))

    out = {}
    for name, fn in (("dynamic_quantize_linear", dql), ("matmul_integer", mmi_prepared), ("matmul_integer_plain", mmi),
                     ("dequantize_linear", dl)):
        fn()  # eager first: sizes the workspace before capture
        ctx.synchronize()
        g = Graph(ctx, lambda fn=fn: [fn() for _ in range(per_graph)])
        us = time_graphs(ctx, [g], reps, 3) * 1e3 / (reps * per_graph)
        g.destroy()
        out[name] = {"us": us}
    out["dynamic_quantize_linear"]["gbs"] = m * k * 5 / (out["dynamic_quantize_linear"]["us"] * 1e-6) / 1e9
    out["matmul_integer"]["tops"] = 2 * m * k * n / (out["matmul_integer"]["us"] * 1e-6) / 1e12
    out["matmul_integer"]["frac_of_int8_peak"] = out["matmul_integer"]["tops"] / INT8_PEAK_TOPS
    out["matmul_integer"]["b"] = "prepared once (tmh_int8_weight_prepare), as the load-time move leaves an initializer"
    out["matmul_integer_plain"]["tops"] = 2 * m * k * n / (out["matmul_integer_plain"]["us"] * 1e-6) / 1e12
    out["dequantize_linear"]["gbs"] = m * k * 5 / (out["dequantize_linear"]["us"] * 1e-6) / 1e9
    log(f"int8 {m}x{k}x{n}: DynamicQuantizeLinear {out['dynamic_quantize_linear']['us']:.1f} us "
        f"({out['dynamic_quantize_linear']['gbs']:.0f} GB/s), MatMulInteger {out['matmul_integer']['us']:.1f} us "
        f"({out['matmul_integer']['tops']:.0f} TOP/s; B as given: {out['matmul_integer_plain']['us']:.1f} us), "
        f"DequantizeLinear {out['dequantize_linear']['us']:.1f} us "
        f"({out['dequantize_linear']['gbs']:.0f} GB/s)")
    for t in (x, xq, xs, xz, bq, bz, y, scale, dq, bw):
        t.free()
    return out


def _torch_graph_us(torch, fn, reps, per_graph):
    """Microseconds per call of fn, from `reps` replays of a torch CUDA graph of `per_graph` calls."""
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * per_graph)


def vendor_gemms(reps, per_graph=10):
    """The vendor library's dense GEMMs at the shapes the bench times, for comparison (torch on
    ROCm calls hipBLASLt), in torch CUDA graphs of `per_graph` calls:
    - int8 2048 x 2048 x 2048 (torch._int_mm, s8 x s8 -> s32, no zero points) with B as [K, N]
      rows and with B k-contiguous (the layout a prepared MatMulInteger weight has), checked
      exactly against an f64 product;
    - f16 x f16 -> f16 at the SmolLM3-3B prefill projections (M = 256 and 2048), weights [N, K]
      as nn.Linear holds them, dense: the f16 GEMM with no dequantization at all, checked against
      an f32 product.
    Opt-in (`--vendor`): it imports torch, whose first import on a fresh machine takes minutes."""
    import torch

    gen = torch.Generator().manual_seed(7)
    out = {"int8": {}, "f16_prefill": {}}
    n = 2048
    a = torch.randint(-128, 128, (n, n), dtype=torch.int8, generator=gen).cuda()
    b = torch.randint(-128, 128, (n, n), dtype=torch.int8, generator=gen).cuda()
    ref = a.double() @ b.double()
    for name, bb in (("b_rows", b), ("b_k_contiguous", b.t().contiguous().t())):
        y = torch._int_mm(a, bb)
        torch.cuda.synchronize()
        if not torch.equal(y.double(), ref):
            raise RuntimeError(f"torch._int_mm ({name}) differs from the exact product")
        us = _torch_graph_us(torch, lambda bb=bb: torch._int_mm(a, bb), reps, per_graph)
        out["int8"][name] = {"us": us, "tops": 2 * n ** 3 / (us * 1e-6) / 1e12}
    log(f"torch._int_mm {n}^3: B rows {out['int8']['b_rows']['us']:.1f} us, "
        f"B k-contiguous {out['int8']['b_k_contiguous']['us']:.1f} us")
    for m in (256, 2048):
        per, flops, total_us = [], 0, 0.0
        for pname, k, nn in SMOLLM3_3B:
            x = torch.randn((m, k), generator=gen).half().cuda()
            w = (torch.randn((nn, k), generator=gen) * 0.02).half().cuda()
            y = torch.nn.functional.linear(x, w)
            ref = x.float() @ w.float().t()
            err = (y.float() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            if not err < 1e-2:
                raise RuntimeError(f"f16 linear {pname} at M={m} is off by {err:.3g} of max|ref|")
            us = _torch_graph_us(torch, lambda x=x, w=w: torch.nn.functional.linear(x, w), reps, per_graph)
            per.append({"projection": pname, "us": us, "tflops": 2 * m * k * nn / (us * 1e-6) / 1e12})
            flops += 2 * m * k * nn
            total_us += us
            del x, w, y, ref
        out["f16_prefill"][str(m)] = {"per_projection": per, "tflops": flops / (total_us * 1e-6) / 1e12}
        log(f"f16 linear (dense) M={m}: " + ", ".join(f"{p['us']:.1f}" for p in per)
            + f" us, {out['f16_prefill'][str(m)]['tflops']:.0f} TFLOP/s")
    return out


# ---------------------------------------------------------------- CPU baseline


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, seconds):
    fn()  # warm-up
    done, t0 = 0, time.perf_counter()
    while True:
        fn()
        done += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            return done, elapsed


def cpu_baseline(seconds=10.0):
    """The reference's EXLA-CPU path restated in C (oracle/oracle.c), on this host's cores:
    - headline: the whole Qwen3-0.6B decode step (28 layers x 7 q4 GEMVs, M = 1) after move/2,
      weights dequantized once to f16 (the scales' type), then an f32-accumulating dot (AVX2 FMA,
      f16 widened by F16C) on every host thread, and the same on one thread;
    - in-graph: the same GEMVs without move/2, dequantizing W in the graph on every call
      (quantized.ex:39-44), on a 4-layer sample;
    - the single f32 op of the CPU configuration (K=1024, N=3072, f32 scales, no zero points),
      after move/2 (f32 weights).
    Reported in the same algorithmic GB/s as the GPU. `seconds` is the time of the headline leg;
    the other legs take a quarter of it each."""
    from oracle import coracle

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    rng = np.random.default_rng(5)
    ws, raw = [], []
    for layer in range(QWEN3_LAYERS):
        for _name, k, n in QWEN3_06B:
            b, sc, zp = make_weight_parts(rng, k, n)
            ws.append((k, n, coracle.dequantize_nbits(b, sc.astype(np.float32), zp, k, n, 4, 32, out_f16=True)))
            if layer < 4:
                raw.append((k, n, b, sc.astype(np.float32), zp))
    a = {k: rng.standard_normal((1, k), dtype=np.float32) for k in (1024, 2048, 3072)}
    step_bytes = QWEN3_LAYERS * sum(nbits_bytes(k, n, 1) for _name, k, n in QWEN3_06B)

    def step(t):
        for k, _n, w16 in ws:
            coracle.gemm(a[k], w16, t)

    done, elapsed = _timed(lambda: step(threads), seconds)
    gbs = done * step_bytes / elapsed / 1e9
    done1, elapsed1 = _timed(lambda: step(1), seconds / 4)
    gbs1 = done1 * step_bytes / elapsed1 / 1e9
    scratch = np.empty((3072, 3072), np.uint16)

    def in_graph():
        for k, n, b, sc, zp in raw:
            coracle.matmul_nbits_in_graph(a[k], b, sc, zp, k, n, 4, 32, True, threads, scratch[:n, :k])

    done_g, elapsed_g = _timed(in_graph, seconds / 4)
    gbs_g = done_g * 4 * sum(nbits_bytes(k, n, 1) for _name, k, n in QWEN3_06B) / elapsed_g / 1e9
    k1, n1 = 1024, 3072
    b1 = rng.integers(0, 256, (n1, k1 // 32, 16), dtype=np.uint8)
    s1 = (np.abs(rng.standard_normal(n1 * k1 // 32, dtype=np.float32)) * 0.01 + 1e-4).astype(np.float32)
    w1 = coracle.dequantize_nbits(b1, s1, None, k1, n1, 4, 32, out_f16=False)
    a1 = rng.standard_normal((1, k1), dtype=np.float32)
    c1_bytes = nbits_bytes(k1, n1, 1, scale_bytes=4, zp=False, a_bytes=4, y_bytes=4)
    done_c, elapsed_c = _timed(lambda: coracle.gemm(a1, w1, threads), seconds / 4)
    c1_us = elapsed_c / done_c * 1e6
    done_c1, elapsed_c1 = _timed(lambda: coracle.gemm(a1, w1, 1), seconds / 8)
    c1_us1 = elapsed_c1 / done_c1 * 1e6
    model = _cpu_model()
    log(f"cpu baseline ({model}, {threads} threads): decode {gbs:.2f} GB/s ({elapsed / done * 1e3:.1f} ms/step), "
        f"1 thread {gbs1:.2f} GB/s; in-graph dequant {gbs_g:.2f} GB/s; single op {c1_us:.1f} us "
        f"({c1_bytes / c1_us / 1e3:.2f} GB/s), 1 thread {c1_us1:.1f} us")
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"whole Qwen3-0.6B decode steps (28 layers x 7 q4 GEMVs, M=1), weights dequantized once to "
                      f"f16, f32-accumulating dot on {threads} threads, {done} steps in {elapsed:.1f} s",
            "cpu_model": model, "nproc": os.cpu_count(), "ms_per_decode_step": elapsed / done * 1e3,
            "one_thread_gbs": gbs1, "in_graph_dequant_gbs": gbs_g,
            "single_op_us": c1_us, "single_op_gbs": c1_bytes / (c1_us * 1e-6) / 1e9, "single_op_one_thread_us": c1_us1}


# ---------------------------------------------------------------- profiling runs

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_gemv_traffic.json")
COPY_BYTES = 256 << 20


def profile_run(ctx, kind, steps, m=1):
    """A short, graph-free run for rocprofv3: `decode` runs the projection sweep at M = m over one
    weight copy plus one 256 MiB device copy (the calibration of the memory counters);
    `prefill` runs the SmolLM3-3B projections at M=2048 (or M = m when m > 1); `moe` the quantized MoE layer; `vocab`
    the lm_head MatMulNBits and the GatherBlockQuantized lookup at the 151936 x 1024 shape; `int8`
    DynamicQuantizeLinear, MatMulInteger and DequantizeLinear at 2048 x 2048 x 2048."""
    global USE_GRAPHS
    USE_GRAPHS = False
    if kind == "decode":
        decode_sweep(ctx, steps, 2, 1, [m])
        src, dst = ctx.empty((COPY_BYTES,), "u8"), ctx.empty((COPY_BYTES,), "u8")
        from transmuter_amd._lib import lib

        for _ in range(3):
            ctx.check(lib().tmh_copy_2d(ctx.handle, dst.ptr, COPY_BYTES, src.ptr, COPY_BYTES, COPY_BYTES, 1, None))
        ctx.synchronize()
    elif kind == "moe":
        moe_ffn(ctx, steps, per_graph=3)
    elif kind == "vocab":
        large_vocab(ctx, steps, per_graph=3)
    elif kind == "int8":
        int8_ops(ctx, steps, per_graph=1)
    else:
        prefill(ctx, steps, [m if m > 1 else 2048])


def summarize(kernel_csv, pmc_dirs):
    """A markdown summary of rocprofv3 output: per-kernel durations (kernel_stats.csv) and,
    for --pmc runs (counter_collection.csv), FETCH_SIZE / WRITE_SIZE per dispatch."""
    import csv
    import glob

    out = []
    if kernel_csv:
        rows = list(csv.DictReader(open(kernel_csv)))
        out.append("| kernel | calls | avg us | min us | max us | total % |")
        out.append("|---|---|---|---|---|---|")
        for r in rows[:12]:
            out.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                       f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    for d in pmc_dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            agg = {}
            for r in csv.DictReader(open(f)):
                key = (r["Kernel_Name"][:70], r["Counter_Name"], r["Grid_Size"])
                agg.setdefault(key, []).append(float(r["Counter_Value"]))
            out.append("")
            out.append("| kernel | counter | grid | dispatches | avg KiB per dispatch |")
            out.append("|---|---|---|---|---|")
            for (k, c, grid), v in sorted(agg.items()):
                out.append(f"| `{k}` | {c} | {grid} | {len(v)} | {sum(v) / len(v):.1f} |")
    return "\n".join(out)


def write_traffic(fetch_dir, write_dir):
    """Writes the decode GEMV's HBM traffic per launch (TRAFFIC_FILE) from two rocprofv3 --pmc runs
    of `--profile decode`, one with FETCH_SIZE and one with WRITE_SIZE. Each counter is scaled by
    what it reads for the 256 MiB calibration copy of the same run (bytes known), and averaged
    over every dispatch of the decode GEMV (k_gemv_dot at M = 1, k_gemv_dec above): the 7
    projections run equally often."""
    import csv
    import glob

    def read(d, counter):
        gemv, copy = [], []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                if "k_gemv_dec" in r["Kernel_Name"] or "k_gemv_dot" in r["Kernel_Name"]:
                    gemv.append(float(r["Counter_Value"]))
                elif "copyBufferRect" in r["Kernel_Name"]:
                    copy.append(float(r["Counter_Value"]))
        if not gemv or not copy:
            raise SystemExit(f"{d}: no decode GEMV or calibration-copy rows for {counter}")
        return sum(gemv) / len(gemv), sum(copy) / len(copy), len(gemv)

    fetch, fetch_copy, n_f = read(fetch_dir, "FETCH_SIZE")
    write, write_copy, n_w = read(write_dir, "WRITE_SIZE")
    copy_kib = COPY_BYTES / 1024
    fs, ws = copy_kib / fetch_copy, copy_kib / write_copy
    hbm = (fetch * fs + write * ws) * 1024
    algo = sum(nbits_bytes(k, n, 1) for _, k, n in QWEN3_06B) / len(QWEN3_06B)
    t = {"what": "HBM bytes per k_gemv_dot launch over the 7 Qwen3-0.6B q4 decode projections at M=1 "
                 "(block 32, f16 scales, packed zero points)",
         "fetch_scale": fs, "write_scale": ws,
         "copy_calibration": {"bytes": COPY_BYTES, "fetch_kib": fetch_copy, "write_kib": write_copy},
         "dispatches": {"fetch_run": n_f, "write_run": n_w},
         "fetch_kib_per_launch": fetch, "write_kib_per_launch": write,
         "hbm_bytes_per_launch": hbm, "algorithmic_bytes_per_launch": algo,
         "traffic_over_algorithmic": hbm / algo}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(t, f, indent=1)
    print(json.dumps(t, indent=1))


def traffic_per_launch():
    """HBM bytes per decode GEMV launch from the committed counter summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    t = json.load(open(TRAFFIC_FILE))
    return t.get("hbm_bytes_per_launch")


# ---------------------------------------------------------------- launch timelines (in-graph kernel times)


def timeline_steps(ctx, records, calls, reps=20, warmup=5, capacity=1 << 22):
    """Times `records` (callables, one step of calls each) as plain HIP graphs, then captures them
    again with the launch timeline on (transmuter_amd.timeline) and replays those stamping graphs
    once each, back to back, after a warm-up. `calls` lists each step's calls as (label, bytes,
    flops). Returns the event-timed ms per step of both runs and, per launch of the stamping
    replays, its kernel, call label and in-kernel time (first wavefront's start to last one's
    end) with the time to the next launch's start."""
    from transmuter_amd.timeline import Timeline

    plain = [Graph(ctx, r) for r in records]
    steps = max(reps, len(plain))
    ms_plain = time_graphs(ctx, plain, steps, warmup) / steps
    tl = Timeline(ctx, capacity)
    tl.begin()
    try:
        stamped = [Graph(ctx, r) for r in records]
    finally:
        log = tl.end()
    if tl.dropped:
        raise RuntimeError(f"the timeline dropped {tl.dropped} launches: raise its capacity")
    for i in range(warmup):
        plain[i % len(plain)].launch()
    ctx.synchronize()
    t = Timer(ctx)
    t.start()
    for g in stamped:
        g.launch()
    ms_stamped = t.stop_ms() / len(stamped)
    launches = tl.launches()
    for g in plain + stamped:
        g.destroy()
    tl.free()
    per_step = len(log) // len(records)
    if per_step * len(records) != len(log):
        raise RuntimeError("the steps launched different numbers of kernels")
    rows = []
    for s in range(len(records)):
        step = launches[s * per_step:(s + 1) * per_step]
        call = -1
        for j, ln in enumerate(step):
            if len(calls) == per_step:  # one entry per stamped launch
                call = j
            elif ln["kernel"] != "k_splitk_reduce":  # one per call; a split-K sum belongs to its GEMM
                call += 1
            label, nbytes, flops = calls[call]
            nxt = step[j + 1]["start_us"] if j + 1 < len(step) else ln["end_us"]
            rows.append({**ln, "step": s, "label": label, "bytes": nbytes, "flops": flops,
                         "to_next_us": nxt - ln["start_us"]})
    return {"ms_per_step": ms_plain, "ms_per_step_stamped": ms_stamped, "steps_stamped": len(records),
            "launches_per_step": per_step, "rows": rows}


def timeline_summary(res):
    """Per (call label, kernel): launches per step, mean in-kernel us, mean launch-to-next-launch
    us, shader clock, and the algorithmic rate over the in-kernel time; per step: the event time
    of plain and stamping replays, the summed in-kernel time and the span from the first start
    to the last end."""
    groups = {}
    for r in res["rows"]:
        groups.setdefault((r["label"], r["kernel"]), []).append(r)
    steps = res["steps_stamped"]
    out = []
    for (label, kernel), rs in groups.items():
        us = float(np.mean([r["us"] for r in rs]))
        nxt = float(np.mean([r["to_next_us"] for r in rs]))
        ghz = [r["ghz"] for r in rs if r.get("ghz")]
        nbytes, flops = rs[0]["bytes"], rs[0]["flops"]
        out.append({"label": label, "kernel": kernel, "per_step": len(rs) / steps, "kernel_us": us,
                    "kernel_us_min": float(min(r["us"] for r in rs)), "kernel_us_max": float(max(r["us"] for r in rs)),
                    "to_next_us": nxt, "ghz": float(np.mean(ghz)) if ghz else None,
                    "gbs_in_kernel": nbytes / (us * 1e-6) / 1e9 if nbytes and kernel != "k_splitk_reduce" else None,
                    "tflops_in_kernel": flops / (us * 1e-6) / 1e12 if flops and kernel != "k_splitk_reduce" else None})
    spans, sums = [], []
    for s in range(steps):
        rs = [r for r in res["rows"] if r["step"] == s]
        spans.append(max(r["end_us"] for r in rs) - min(r["start_us"] for r in rs))
        sums.append(sum(r["us"] for r in rs))
    return {"ms_per_step": res["ms_per_step"], "ms_per_step_stamped": res["ms_per_step_stamped"],
            "launches_per_step": res["launches_per_step"], "steps_stamped": steps,
            "kernel_us_per_step": float(np.mean(sums)), "span_us_per_step": float(np.mean(spans)), "kernels": out}


def timeline_markdown(title, command, parts, notes):
    lines = [f"# {title}", "", "Command (MI355X, one GPU):", "", "```", command, "```", ""]
    lines += notes + [""]
    for name, s in parts:
        lines += [f"## {name}", "",
                  f"- event-timed step, plain graphs: {s['ms_per_step'] * 1e3:.1f} us; stamping graphs: "
                  f"{s['ms_per_step_stamped'] * 1e3:.1f} us ({s['steps_stamped']} steps stamped, "
                  f"{s['launches_per_step']} launches per step)",
                  f"- per step: in-kernel time summed over the launches {s['kernel_us_per_step']:.1f} us; first "
                  f"start to last end {s['span_us_per_step']:.1f} us", "",
                  "| call | kernel | per step | in-kernel us (mean, min-max) | start to next start us | "
                  "shader GHz | GB/s in-kernel | TFLOP/s in-kernel |",
                  "|---|---|---|---|---|---|---|---|"]
        for k in s["kernels"]:
            gbs = f"{k['gbs_in_kernel']:.0f}" if k["gbs_in_kernel"] else "-"
            tf = f"{k['tflops_in_kernel']:.1f}" if k["tflops_in_kernel"] else "-"
            ghz = f"{k['ghz']:.2f}" if k["ghz"] else "-"
            lines.append(f"| {k['label']} | `{k['kernel']}` | {k['per_step']:g} | {k['kernel_us']:.2f} "
                         f"({k['kernel_us_min']:.2f}-{k['kernel_us_max']:.2f}) | {k['to_next_us']:.2f} | {ghz} | "
                         f"{gbs} | {tf} |")
        lines.append("")
    lines += ["```json", json.dumps({name: s for name, s in parts}, indent=1), "```", ""]
    return "\n".join(lines)


def decode_weights(ctx, sets, rng):
    from transmuter_amd import PackedWeight

    weights = []
    for _s in range(sets):
        weights.append([[PackedWeight.upload(ctx, *make_weight_parts(rng, k, n), k=k, n=n, bits=4, block_size=32,
                                             weight_dtype="f16") for _name, k, n in QWEN3_06B]
                        for _layer in range(QWEN3_LAYERS)])
    return weights


def timeline_decode(ctx, sets=4, steps=8, m=1, floors=True):
    """The headline decode step (196 GEMVs at M = m over rotating weight copies) with the launch
    timeline, and the same step's floors: an empty kernel per projection, a plain read of each
    projection's packed weights, and a plain read of all its bytes (weights, scales, zero points)."""
    from transmuter_amd._lib import lib

    rng = np.random.default_rng(20260101)
    weights = decode_weights(ctx, sets, rng)
    a = {k: ctx.put(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)) for k in (1024, 2048, 3072)}
    y = {n: ctx.empty((m, n), "f16") for n in (1024, 2048, 3072)}
    sink = ctx.empty((16,), "u8")
    calls = [(f"{name} {k}->{n}", nbits_bytes(k, n, m), 2 * m * k * n) for _layer in range(QWEN3_LAYERS)
             for name, k, n in QWEN3_06B]
    parts = []
    gemv = timeline_steps(ctx, [lambda s=s: [matmul_call(ctx, w, a[w.k], y[w.n], m) for layer in weights[s % sets]
                                             for w in layer] for s in range(steps)], calls)
    parts.append((f"decode GEMVs, M={m}", timeline_summary(gemv)))
    if floors:
        fl = [("empty kernel", lambda w: lib().tmh_floor_empty(ctx.handle, 256, None)),
              ("plain read of the packed weights", lambda w: lib().tmh_floor_read(ctx.handle, w.handle, sink.ptr, None)),
              ("plain read of weights, scales and zero points",
               lambda w: lib().tmh_floor_read_all(ctx.handle, w.handle, sink.ptr, None))]
        for name, fn in fl:
            res = timeline_steps(ctx, [lambda s=s, fn=fn: [ctx.check(fn(w)) for layer in weights[s % sets] for w in layer]
                                       for s in range(steps)], [(c[0], c[1], 0) for c in calls])
            parts.append((f"floor: {name}", timeline_summary(res)))
    for ws in weights:
        for layer in ws:
            for w in layer:
                w.free()
    return parts


def timeline_vocab(ctx, per_graph=12):
    """lm_head (151936 x 1024, M = 1 and 8) over 12 rotating weight copies, the plain read of all
    its bytes, the [8, 512] vocabulary gather and the store-only launch of the gather's output."""
    from transmuter_amd import PackedWeight
    from transmuter_amd._lib import F16, S64, U8, lib

    rng = np.random.default_rng(4)
    vocab, hidden = 151936, 1024
    b, sc, zp = make_weight_parts(rng, hidden, vocab)
    ws = [PackedWeight.upload(ctx, b, sc, zp, k=hidden, n=vocab, bits=4, block_size=32, weight_dtype="f16")]
    ws += [PackedWeight.concat([ws[0]]) for _ in range(-(-ROTATE_BYTES // ws[0].device_bytes()) - 1)]
    parts = []
    for m in (1, 8):
        a = ctx.put(rng.standard_normal((m, hidden), dtype=np.float32).astype(np.float16))
        y = ctx.empty((m, vocab), "f16")
        res = timeline_steps(ctx, [lambda s=s: [matmul_call(ctx, ws[(s * per_graph + i) % len(ws)], a, y, m)
                                                for i in range(per_graph)] for s in range(2)],
                             [(f"lm_head M={m}", nbits_bytes(hidden, vocab, m), 2 * m * hidden * vocab)] * per_graph)
        parts.append((f"lm_head 151936x1024, M={m}", timeline_summary(res)))
    sink = ctx.empty((16,), "u8")
    all_bytes = ws[0].device_bytes()
    res = timeline_steps(ctx, [lambda s=s: [ctx.check(lib().tmh_floor_read_all(ctx.handle, ws[(s * per_graph + i) % len(ws)]
                                                                               .handle, sink.ptr, None))
                                            for i in range(per_graph)] for s in range(2)],
                         [("plain read of the weight's bytes", all_bytes, 0)] * per_graph)
    parts.append(("floor: plain read of all lm_head bytes (weights, scales, zero points)", timeline_summary(res)))
    for w in ws:
        w.free()
    tables = [(ctx.put(b.reshape(vocab, -1)), ctx.put(sc.reshape(vocab, -1)), ctx.put(zp.reshape(vocab, -1)))
              for _ in range(2)]
    ids = [ctx.put(rng.integers(0, vocab, (8, 512)).astype(np.int64)) for _ in range(per_graph)]
    rows = ctx.empty((8, 512, hidden), "f16")

    def gathers(s):
        for i in range(per_graph):
            table, scales, zps = tables[(s + i) % 2]
            ctx.check(lib().tmh_gather_block_quantized(ctx.handle, table.ptr, U8, vocab, hidden // 2, ids[i].ptr, S64,
                                                       4096, scales.ptr, F16, hidden // 32, zps.ptr, U8, 4, rows.ptr,
                                                       None))

    g_bytes = 4096 * (hidden // 2 + hidden // 32 * 2 + hidden // 64 + 8) + 4096 * hidden * 2
    res = timeline_steps(ctx, [lambda s=s: gathers(s) for s in range(2)], [("gather [8, 512]", g_bytes, 0)] * per_graph)
    parts.append(("GatherBlockQuantized [8, 512] ids of 151936 x 1024", timeline_summary(res)))
    out_bytes = 4096 * hidden * 2
    res = timeline_steps(ctx, [lambda: [ctx.check(lib().tmh_floor_write(ctx.handle, rows.ptr, out_bytes, None))
                                        for _ in range(per_graph)]] * 2, [("store-only", out_bytes, 0)] * per_graph)
    parts.append(("floor: the gather's 8 MiB of output stores alone", timeline_summary(res)))
    return parts


def timeline_prefill(ctx, ms=(256, 2048), per_graph=4):
    """The SmolLM3-3B prefill projections at each M, each call on its own weight copy."""
    from transmuter_amd import PackedWeight

    rng = np.random.default_rng(3)
    parts = []
    for name, k, n in SMOLLM3_3B:
        b, sc, zp = make_weight_parts(rng, k, n, bs=128, scale_mul=0.005)
        w0 = PackedWeight.upload(ctx, b, sc, zp, k=k, n=n, bits=4, block_size=128, weight_dtype="f16")
        copies = [w0] + [PackedWeight.concat([w0]) for _ in range(max(1, -(-ROTATE_BYTES // w0.device_bytes())) - 1)]
        for m in ms:
            a = ctx.put(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16))
            y = ctx.empty((m, n), "f16")
            matmul_call(ctx, copies[0], a, y, m)  # sizes the split-K workspace before capture
            ctx.synchronize()
            steps = min(4, max(1, len(copies) // per_graph))
            res = timeline_steps(ctx, [lambda s=s: [matmul_call(ctx, copies[(s * per_graph + i) % len(copies)], a, y, m)
                                                    for i in range(per_graph)] for s in range(steps)],
                                 [(f"{name} M={m}", nbits_bytes(k, n, m, bs=128), 2 * m * k * n)] * per_graph)
            parts.append((f"prefill {name}, M={m}", timeline_summary(res)))
            a.free()
            y.free()
        for w in copies:
            w.free()
    return parts


def timeline_moe(ctx, sets=3, steps=6):
    """The QMoE layer of moe_ffn, one call per step over `sets` rotating copies of its experts:
    routing, grouping by expert, the grouped expert products (fc1 and fc3 with the SwiGLU in one
    launch, then fc2) and the weighted sum over each token's slots."""
    import ctypes

    from transmuter_amd._lib import F16, F32, lib
    from transmuter_amd.moe import ExpertWeight

    rng = np.random.default_rng(6)
    experts, k, hidden, inter, tokens = 128, 8, 2048, 768, 512

    def expert_weight(n, kk):
        packed = rng.integers(0, 256, (experts, n, kk // 2), dtype=np.uint8)
        scales = (np.abs(rng.standard_normal((experts, n, kk // 32), dtype=np.float32)) * 0.01 + 1e-4).astype(np.float16)
        return ExpertWeight.upload(ctx, packed, scales, None, bits=4, block_size=32, dtype="f16")

    def device_copy(w):
        handle = ctypes.c_void_p()
        ctx.check(lib().tmh_weight_concat_nbits(ctx.handle, (ctypes.c_void_p * 1)(w.handle.value), 1,
                                                ctypes.byref(handle)))
        return ExpertWeight(ctx, handle, w.experts, w.n, w.k, w.bits, w.dtype)

    first = (expert_weight(inter, hidden), expert_weight(inter, hidden), expert_weight(hidden, inter))
    layers = [first] + [tuple(device_copy(w) for w in first) for _ in range(sets - 1)]
    x = ctx.put(rng.standard_normal((tokens, hidden), dtype=np.float32).astype(np.float16))
    router = ctx.put(rng.standard_normal((tokens, experts), dtype=np.float32))
    y = ctx.empty((tokens, hidden), "f16")

    def call(i):
        fc1, fc3, fc2 = layers[i % len(layers)]
        ctx.check(lib().tmh_qmoe(ctx.handle, x.ptr, F16, tokens, hidden, router.ptr, F32, experts, k, fc1.handle, None,
                                 fc2.handle, None, fc3.handle, None, F16, 4, 0, 1.0, 0.0, 0.0, y.ptr, None))

    call(0)  # sizes the workspace before capture
    ctx.synchronize()
    wb = experts * hidden * inter * (0.5 + 2 / 32)  # one projection's expert weights and scales
    rows = tokens * k
    calls = [("routing (top-8 of 128)", tokens * experts * 4 + rows * 8, 0),
             ("grouping by expert", rows * 4 * 4 + experts * 12, 0),
             ("fc1 + fc3 (SwiGLU)", 2 * wb + tokens * hidden * 2 + rows * inter * 2, 2 * 2 * rows * hidden * inter),
             ("fc2", wb + rows * inter * 2 + rows * hidden * 2, 2 * rows * hidden * inter),
             ("weighted sum over the slots", rows * hidden * 2 + tokens * hidden * 2 + rows * 12, 0)]
    res = timeline_steps(ctx, [lambda s=s: call(s) for s in range(steps)], calls)
    for layer in layers:
        for w in layer:
            w.free()
    return [("QMoE 128 experts, top-8, 2048/768, 512 tokens", timeline_summary(res))]


TIMELINE_NOTES = [
    "In-kernel times come from the stamping build of each kernel (transmuter_amd.timeline): every",
    "wavefront writes the 100 MHz real-time counter at its start and, after its memory accesses have",
    "completed, at its end; a launch's time is its first wavefront's start to its last one's end, read",
    "from the same HIP graph replays that are timed with events (the stamping graphs replay once each,",
    "back to back, after a warm-up of the plain graphs). 'start to next start' is the time from a",
    "launch's first wavefront to the next launch's first wavefront inside the replay. The shader clock",
    "is the cycle counter over the real-time counter across the launch's wavefronts. Rates count",
    "algorithmic bytes and FLOPs.",
]


# ---------------------------------------------------------------- main


def main():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--sets", type=int, default=4, help="weight copies the decode steps rotate over")
    p.add_argument("--quick", action="store_true", help="decode M=1 only")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-graph", action="store_true", help="launch each call on the stream, no HIP graphs")
    p.add_argument("--sections", default="all",
                   help="comma list of parts to run besides the M=1 decode headline: decode (M=4/8/16 and merged), "
                        "single, prefill, vocab, moe, int8, cpu (default all)")
    p.add_argument("--profile", choices=["decode", "prefill", "moe", "vocab", "int8"], help="a short graph-free run for rocprofv3")
    p.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="write the decode GEMV's HBM bytes per launch from two --pmc runs of --profile decode")
    p.add_argument("--profile-m", type=int, default=1, help="rows of A for --profile decode (and prefill, when above 1)")
    p.add_argument("--vendor", action="store_true",
                   help="time the vendor library's dense int8 and f16 GEMMs (torch) at the bench's shapes and exit")
    p.add_argument("--summarize", nargs="*", metavar="PATH",
                   help="print a markdown summary of rocprofv3 output: a kernel_stats.csv, then --pmc directories")
    p.add_argument("--timeline", choices=["decode", "vocab", "prefill", "moe"],
                   help="time a workload's kernels inside its graph replays (stamping builds) and write markdown")
    p.add_argument("--out", help="file the --timeline markdown goes to (default: timeline_KIND.md in the working directory)")
    p.add_argument("--no-timeline", action="store_true", help="skip the in-graph kernel times of the headline")
    args = p.parse_args()
    if args.traffic:
        write_traffic(*args.traffic)
        return
    if args.summarize is not None:
        paths = args.summarize
        kernel_csv = paths[0] if paths and paths[0].endswith(".csv") else None
        print(summarize(kernel_csv, paths[1:] if kernel_csv else paths))
        return
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    if USE_GRAPHS and not args.profile and not args.vendor and rocprof_domains():
        print(f"bench.py: {GRAPHS_UNDER_TRACER}; found {', '.join(rocprof_domains())}. Use --profile KIND "
              "(graph-free launches) or --no-graph under the profiler.", file=sys.stderr)
        sys.exit(3)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path runs on one GPU, "
              "and its multi-GPU sharding is a design, not a measured run)", file=sys.stderr)
        sys.exit(2)

    if args.vendor:
        # In a process of its own: torch brings its own HIP runtime, which finds no GPU once this
        # library's runtime holds the device (run `--sections int8,prefill` beside it).
        print(json.dumps({"vendor": vendor_gemms(20)}))
        return

    from transmuter_amd import Context

    ctx = Context(0)
    if args.profile:
        profile_run(ctx, args.profile, args.steps, args.profile_m)
        ctx.close()
        return
    if args.timeline:
        parts = {"decode": lambda: timeline_decode(ctx, sets=args.sets), "vocab": lambda: timeline_vocab(ctx),
                 "prefill": lambda: timeline_prefill(ctx), "moe": lambda: timeline_moe(ctx)}[args.timeline]()
        title = {"decode": "Qwen3-0.6B q4 decode step (M=1) and its floors, timed inside the graph replays",
                 "vocab": "151936 x 1024 lm_head and vocabulary gather, timed inside the graph replays",
                 "prefill": "SmolLM3-3B q4 prefill projections, timed inside the graph replays",
                 "moe": "Qwen3-30B-A3B QMoE layer (512 tokens), timed inside the graph replays"}[args.timeline]
        out = args.out or f"timeline_{args.timeline}.md"
        if os.path.dirname(out):
            os.makedirs(os.path.dirname(out), exist_ok=True)
        with open(out, "w") as f:
            f.write(timeline_markdown(title, f"python bench.py --timeline {args.timeline}", parts, TIMELINE_NOTES))
        log(f"wrote {out}")
        ctx.close()
        return
    global STAMP_HEADLINE
    STAMP_HEADLINE = not args.no_timeline
    parts = {"decode", "single", "prefill", "vocab", "moe", "int8", "cpu"} if args.sections == "all" \
        else set(args.sections.split(","))
    if args.quick:
        parts = set()
    ms = [1, 4, 8, 16] if "decode" in parts else [1]
    dec = decode_sweep(ctx, args.steps, args.warmup, args.sets, ms, full_step=True)
    dec_merged = decode_sweep(ctx, args.steps, args.warmup, args.sets, ms, merged=True) if "decode" in parts else {}
    extra = {}
    if "single" in parts:
        extra["single_op"] = single_op(ctx, 10)
    if "prefill" in parts:
        extra["prefill"] = prefill(ctx, 20, [256, 2048])
        # The other activation types on the same shapes: bf16 (bf16 MFMA) and f32 (hi + lo splits).
        extra["prefill_bf16"] = prefill(ctx, 10, [256, 2048], dtype="bf16")
        extra["prefill_f32"] = prefill(ctx, 6, [256, 2048], dtype="f32")
    if "vocab" in parts:
        extra["large_vocab"] = large_vocab(ctx, 50)
    if "moe" in parts:
        extra["moe"] = moe_ffn(ctx, 20)
    if "int8" in parts:
        extra["int8"] = int8_ops(ctx, 20)
    head = dec[1]
    roofline = {
        "bound": "hbm", "kernel": "k_gemv_dot<4,zp>", "achieved": head["bytes_per_launch"] / (head["us_per_launch"] * 1e-6) / 1e9,
        "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "traffic": traffic_per_launch(),
    }
    roofline["frac"] = roofline["achieved"] / HBM_PEAK_GBS
    for key in ("launch_floor_us", "read_floor_us", "read_floor_gbs"):
        roofline[key] = head.get(key)
    if head.get("read_floor_us"):
        # The GEMV's launch time against a launch that only reads the same packed weights.
        roofline["read_floor_over_launch"] = head["read_floor_us"] / head["us_per_launch"]
    if head.get("timeline"):
        # The same kernel inside the replays (launch timeline): first wavefront's start to last
        # one's end, averaged over its launches; achieved_in_kernel counts the same bytes over it.
        tls = head["timeline"]
        gemv = [k for k in tls["kernels"] if k["kernel"] in ("k_gemv_dot", "k_gemv_dec")]
        n = sum(k["per_step"] for k in gemv)
        kernel_us = sum(k["kernel_us"] * k["per_step"] for k in gemv) / n
        roofline.update({
            "kernel_us_in_graph": kernel_us,
            "start_to_next_start_us_in_graph": sum(k["to_next_us"] * k["per_step"] for k in gemv) / n,
            "achieved_in_kernel": head["bytes_per_launch"] / (kernel_us * 1e-6) / 1e9,
            "shader_ghz": sum((k["ghz"] or 0) * k["per_step"] for k in gemv) / n,
            "stamped_ms_per_step": tls["ms_per_step_stamped"],
            "kernel_us_per_step_in_graph": tls["kernel_us_per_step"],
        })
    cpu = None if args.no_cpu or "cpu" not in parts else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": "MatMulNBits q4: GB/s @M=1 and TFLOP/s @M=2048, % of MI355X roofline",
        "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded random q4 weights, N(0,1) activations)",
        "config": {"workload": "Qwen3-0.6B q4 decode projection sweep (28 layers x q,k,v,o,gate,up,down; block 32; "
                               "f16 A and scales; packed zero points), M=1, 4 rotating weight copies",
                   "M": 1, "layers": QWEN3_LAYERS, "weight_copies": args.sets, "parallelism": "single GPU"},
        "tokens_per_s": head["tokens_per_s"],
        "decode_sweep": {str(m): {k: v for k, v in r.items() if k in ("gbs", "tflops", "ms_per_step", "us_per_launch",
                                                                      "tokens_per_s", "ms_per_step_with_lm_head",
                                                                      "tokens_per_s_with_lm_head", "single_launch_us")}
                         for m, r in dec.items()},
        "tokens_per_s_with_lm_head": head.get("tokens_per_s_with_lm_head"),
        "single_launch_us": head.get("single_launch_us"),
        "eager_tokens_per_s": head.get("eager_tokens_per_s"),
        "decode_merged_qkv_gateup": {str(m): {k: v for k, v in r.items() if k in ("gbs", "ms_per_step", "us_per_launch",
                                                                                  "tokens_per_s", "launch_floor_us",
                                                                                  "read_floor_us", "read_floor_gbs")}
                                     for m, r in dec_merged.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if "prefill" in extra:
        line["prefill"] = {str(m): v for m, v in extra["prefill"].items()}
        line["prefill_tflops_M2048"] = extra["prefill"][2048]["tflops"]
        line["prefill_frac_M2048"] = extra["prefill"][2048]["tflops"] / MFMA_F16_PEAK_TFLOPS
        for dt in ("bf16", "f32"):
            line[f"prefill_{dt}"] = {str(m): v for m, v in extra[f"prefill_{dt}"].items()}
            line[f"prefill_{dt}_over_f16_M2048"] = extra[f"prefill_{dt}"][2048]["tflops"] / extra["prefill"][2048]["tflops"]
    for key, name in (("large_vocab", "large_vocab"), ("single_op", "single_op_f32_k1024_n3072"), ("moe", "moe"),
                      ("int8", "int8")):
        if key in extra:
            line[name] = extra[key]
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
