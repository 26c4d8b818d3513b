#!/usr/bin/env python3
"""Benchmark of the AccelEP hot path on one MI355X: the claimed MatMul on a packed
constant int8 weight (accel::MatMulQuantized) and its fp32-MFMA forms.

Headline (`value`): the int8-weight decode GEMV, X fp32 [1, 4096] @ W int8 [4096, 14336]
with a per-column fp32 scale, in algorithmic GB/s. Eight device copies of W (470 MB, more
than the 256 MB Infinity Cache) are used round robin so every step streams W from HBM.
A step is one accel_hip_matmul_quantized call; the K timed steps are replayed from HIP
graphs of up to 200 steps, timed between two HIP events on the library stream.

Secondary lines (same JSON object, "secondary"): the GEMV at M = 4 and 16, the fp32 MLP
(Gemm+bias+Gelu, Gemm+bias+residual, fused epilogues) in TFLOP/s, the int8 prefill GEMM
M=2048 K=4096 N=14336 with fused RMSNormalization in TFLOP/s, and the cache-warm GEMV.

cpu_baseline: the reference's own MatMulQuantized (AccelEP src/sim_device.cc, compiled by
oracle/Makefile into oracle/_ref) on the same M = 1 workload, single thread on the host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "int8-W GEMV HBM GB/s + GEMM fp32-MFMA TFLOP/s (% peak); decode tok/s"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
# The int8-weight GEMM runs each fp32 product as three exact bf16 MFMA passes (activation split
# into hi + mid + lo): its roofline is a third of the dense bf16 peak.
BF16X3_PEAK_TFLOPS = 2500.0 / 3
K_DIM, N_DIM = 4096, 14336
COPIES = 8
C1_SHAPE = (4, 576, 1536)  # X[4,576] @ int8 W[576,1536]
MLP_SHAPE = (256, 1024, 4096)  # X[256,1024] -> 4096 -> 1024


def gemv_bytes(m, k=K_DIM, n=N_DIM):
    """Algorithmic HBM bytes of one GEMV: int8 W once, fp32 scale, X read, C written."""
    return k * n + 4 * n + 4 * m * k + 4 * m * n


TRAFFIC_PROFILE = ROOT / "profiles" / "gemv_q8_m1_4096x14336_pmc.md"


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed FETCH_SIZE/WRITE_SIZE
    profile (rocprofv3 --pmc runs, scaled by a streaming kernel of known traffic), or None."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    def __init__(self):
        from accelep_amd.capi import Epilogue, QuantPlane, check, lib
        from accelep_amd.device import DeviceArray, quant_plane

        self.L = lib()
        self.check = check
        self.Epilogue = Epilogue
        self.QuantPlane = QuantPlane
        self.DeviceArray = DeviceArray
        self.quant_plane = quant_plane
        check(self.L.accel_hip_init())
        self.arch = self.L.accel_hip_device_arch().decode()

    def sync(self):
        self.check(self.L.accel_hip_synchronize())

    def graph(self, fn, count):
        """Captures `count` calls of fn(i) into one executable graph."""
        self.check(self.L.accel_hip_capture_begin())
        try:
            for i in range(count):
                fn(i)
        finally:
            g = C.c_void_p()
            self.check(self.L.accel_hip_capture_end(C.byref(g)))
        return g

    def elapsed(self):
        ms = self.L.accel_hip_event_elapsed_ms(0, 1)
        if ms < 0:
            raise RuntimeError(self.L.accel_hip_last_error().decode())
        return ms

    def time_in_graph(self, step, lead_len, steps):
        """Times `steps` calls of step(i) between two event records captured in one graph after
        `lead_len` untimed calls (whole weight rotations): the graph's launch and the lead-in
        fall before the start event. The first replay uploads the graph and sizes the clock
        warm-up; then the graph is replayed back to back for at least CLOCK_WARM_MS of GPU time
        and the last replay's event pair, which holds exactly `steps` steps, is the result.
        Returns elapsed ms."""
        self.check(self.L.accel_hip_capture_begin())
        try:
            for i in range(lead_len):
                step(i)
            self.check(self.L.accel_hip_event_record(0))
            for i in range(steps):
                step(i)
            self.check(self.L.accel_hip_event_record(1))
        finally:
            g = C.c_void_p()
            self.check(self.L.accel_hip_capture_end(C.byref(g)))
        try:
            self.check(self.L.accel_hip_graph_launch(g, 1))
            replay_ms = self.elapsed() * (lead_len + steps) / steps
            self.check(self.L.accel_hip_graph_launch(g, warm_replays(replay_ms) + 1))
            return self.elapsed()
        finally:
            self.L.accel_hip_graph_destroy(g)

    def time_graph(self, graphs_and_reps, lead=None, warm=None):
        """Event-timed replay: list of (graph, reps); returns elapsed ms.

        `lead`, a graph replayed once (untimed) just before the start event, keeps the GPU busy
        while the host submits the start event, the timed graphs and the end event: the timed
        interval then holds the steps and not the host's submission latency (about 12 us,
        which over 20 steps of a 10.5 us GEMV would read as 0.6 us a step). `warm`, a (graph,
        reps) pair replayed untimed before the lead, brings the clocks to their steady state."""
        self.sync()
        if warm is not None:
            self.check(self.L.accel_hip_graph_launch(warm[0], warm[1]))
        if lead is not None:
            self.check(self.L.accel_hip_graph_launch(lead, 1))
        self.check(self.L.accel_hip_event_record(0))
        for g, reps in graphs_and_reps:
            if reps:
                self.check(self.L.accel_hip_graph_launch(g, reps))
        self.check(self.L.accel_hip_event_record(1))
        ms = self.L.accel_hip_event_elapsed_ms(0, 1)
        if ms < 0:
            raise RuntimeError(self.L.accel_hip_last_error().decode())
        return ms


GRAPHS = True  # --no-graph: launch every step directly (profiler counter runs see each dispatch)
LEAD_STEPS = 4  # untimed steps replayed right before the start event (rounded up to whole rotations)
# Untimed GPU work replayed back to back right before a timed replay. From idle, the first
# milliseconds of a memory-bound stream run slow: the m = 1 GEMV's first replay of 400 steps read
# 10.4-10.6 us a step where later ones read 10.2 (one box, same graph), and a lone replay of 20
# steps after the short warm-up ran slower still. 50 ms of the same steps takes that out.
CLOCK_WARM_MS = 50.0


def warm_replays(replay_ms):
    """Replays of a graph of `replay_ms` that cover CLOCK_WARM_MS (at most 20000)."""
    return int(min(20000, max(1, -(-CLOCK_WARM_MS // max(replay_ms, 1e-3)))))


def timed_steps(hip, step, steps, warmup, period=200, rotation=1):
    """Warms up, captures the timed calls into HIP graphs, times exactly `steps` steps.

    Step i reads weight copy i % rotation. The warm-up calls every copy at least once, so
    each is staged (the GEMV's first use of a weight builds its tiled copy, which the library
    refuses inside a capture; the fp32 GEMM stages a weight's bf16 parts on its second use)
    and the workspaces have their final size before anything is captured. A lead-in of whole rotations (at least 4 steps) runs untimed right before the
    start event and ends on the last copy, so the timed steps walk the copies in order and a
    copy is never read again before the other copies (> 256 MB) have streamed through the
    cache.
    - Up to 400 steps: one graph holds the lead-in, the start event record, exactly `steps`
      steps and the end event record (records inside a capture become timeable event nodes),
      replayed once untimed (its first replay uploads it), then back to back for the clock
      warm-up (CLOCK_WARM_MS), the last replay timed. Neither the host's submission nor the
      graph's launch on the GPU (about 5 us) falls inside the interval.
    - More steps: graphs of `period` nodes (a whole number of rotations) plus one for the
      rest, each replayed once untimed; then the first of them for the clock warm-up, the
      lead-in graph and the timed replays back to back between two events on the stream (one
      graph launch per `period` steps stays in)."""
    for i in range(max(warmup, rotation, 1)):
        step(i)
    hip.sync()
    lead_len = rotation * -(-LEAD_STEPS // rotation)
    if not GRAPHS:
        for i in range(lead_len):
            step(i)
        hip.check(hip.L.accel_hip_event_record(0))
        for i in range(steps):
            step(i)
        hip.check(hip.L.accel_hip_event_record(1))
        return hip.L.accel_hip_event_elapsed_ms(0, 1)
    if steps <= 400:
        return hip.time_in_graph(step, lead_len, steps)
    lead = hip.graph(step, lead_len)
    period = min(period, steps)
    if period > rotation:
        period -= period % rotation
    plan = [(hip.graph(step, period), steps // period)]
    if steps % period:
        plan.append((hip.graph(step, steps % period), 1))
    graphs = [lead] + [g for g, _ in plan]
    try:
        for g in graphs:  # the first replay of a graph uploads it
            hip.check(hip.L.accel_hip_graph_launch(g, 1))
        period_ms = hip.time_graph([(plan[0][0], 1)])
        return hip.time_graph(plan, lead=lead, warm=(plan[0][0], warm_replays(period_ms)))
    finally:
        for g in graphs:
            hip.L.accel_hip_graph_destroy(g)


def bench_gemv(hip, m, steps, warmup, copies, rng):
    """Returns (ms_per_step, GB/s) for the int8 GEMV at this M over `copies` weight copies."""
    q_host = rng.integers(-127, 128, size=K_DIM * N_DIM, dtype=np.int8)
    scale = hip.DeviceArray.from_numpy(rng.uniform(1e-3, 1e-2, size=N_DIM).astype(np.float32))
    weights = [hip.DeviceArray.from_numpy(q_host) for _ in range(copies)]
    planes = [hip.quant_plane(w, scale, None, [K_DIM, N_DIM], 1) for w in weights]
    x = hip.DeviceArray.from_numpy(rng.standard_normal((m, K_DIM)).astype(np.float32))
    out = hip.DeviceArray((m, N_DIM))

    def step(i):
        hip.check(hip.L.accel_hip_matmul_quantized(x.ptr, None, None, C.byref(planes[i % copies]), out.ptr, m, K_DIM,
                                                   N_DIM))

    ms = timed_steps(hip, step, steps, warmup, period=25 * copies, rotation=copies)
    per = ms / steps
    return per, gemv_bytes(m) / (per * 1e-3) / 1e9


def bench_mlp(hip, steps, warmup, rng):
    """fp32 MLP X[256,1024] -> Gemm(1024x4096)+bias -> Gelu -> Gemm(4096x1024)+bias + X.

    Two fused calls per step (bias+gelu, bias+residual epilogues in registers)."""
    m, d, h = MLP_SHAPE
    x, w1, b1, w2, b2 = (hip.DeviceArray.from_numpy(v) for v in mlp_inputs(rng))
    hid = hip.DeviceArray((m, h))
    y = hip.DeviceArray((m, d))
    e1 = hip.Epilogue(alpha=1.0, beta=1.0, bias=b1.ptr, bias_rank=1, activation=2)
    e1.bias_shape[0] = h
    e2 = hip.Epilogue(alpha=1.0, beta=1.0, bias=b2.ptr, bias_rank=1, activation=0, residual=x.ptr)
    e2.bias_shape[0] = d

    def step(i):
        hip.check(hip.L.accel_hip_matmul_fused(x.ptr, w1.ptr, hid.ptr, m, d, h, C.byref(e1)))
        hip.check(hip.L.accel_hip_matmul_fused(hid.ptr, w2.ptr, y.ptr, m, h, d, C.byref(e2)))

    ms = timed_steps(hip, step, steps, warmup)
    per = ms / steps
    flops = 2 * m * d * h * 2
    return per, flops / (per * 1e-3) / 1e12


def bench_prefill(hip, steps, warmup, rng):
    """int8 prefill GEMM X[2048,4096] @ W int8[4096,14336] (per-column scale) + RMSNormalization
    (eps 1e-5, gamma ~ N(1, 0.1)) of the output rows, written in place."""
    m, k, n = 2048, K_DIM, N_DIM
    q = hip.DeviceArray.from_numpy(rng.integers(-127, 128, size=k * n, dtype=np.int8))
    scale = hip.DeviceArray.from_numpy(rng.uniform(1e-3, 1e-2, size=n).astype(np.float32))
    plane = hip.quant_plane(q, scale, None, [k, n], 1)
    x = hip.DeviceArray.from_numpy(rng.standard_normal((m, k)).astype(np.float32))
    g = hip.DeviceArray.from_numpy((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    out = hip.DeviceArray((m, n))
    e = hip.Epilogue(alpha=1.0, beta=1.0, rms_weight=g.ptr, rms_eps=1e-5, rms_out=out.ptr)

    def step(i):
        hip.check(hip.L.accel_hip_matmul_quantized_fused(x.ptr, None, None, C.byref(plane), out.ptr, m, k, n,
                                                         C.byref(e)))

    ms = timed_steps(hip, step, steps, warmup)
    per = ms / steps
    return per, 2 * m * k * n / (per * 1e-3) / 1e12


SMOL = dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, intermediate=1536, context=640, eps=1e-5,
            rope_theta=100000.0)
# Bytes one decode token reads at least once: int8 layer weights 106,168,320 + their scales
# 622,080 + int8 LM head 28,311,552 + norms 140,544 + the K/V rows of 30 layers at the mean
# position of a 512 + 128 generation (46,080 B per position, 576 positions on average).
LLAMA_DECODE_BYTES = 106_168_320 + 622_080 + 28_311_552 + 140_544 + 46_080 * 576


def llama_q8_weights(cfg, rng):
    """SmolLM2-135M-shape random-init weights in Hugging Face layout ([out, in] matrices):
    every linear weight and the tied embedding / LM head ~ N(0, 0.02), quantized per output row
    (s = max|w| / 127, q = rint(w / s)); norm weights ~ N(1, 0.1). Yields (kind, layer, q, s)
    for the int8 matrices and (kind, layer, w, None) for the norms."""
    H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    hd = H // cfg["heads"]

    def q8(rows, cols):
        w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        s = (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32)
        s[s == 0] = 1
        return np.rint(w / s[:, None]).clip(-127, 127).astype(np.int8), s

    def norm():
        return (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)

    emb_q, emb_s = q8(V, H)
    yield 1, -1, emb_q, emb_s
    yield 3, -1, emb_q, emb_s  # LM head tied to the embedding
    yield 2, -1, norm(), None
    shapes = {6: (cfg["heads"] * hd, H), 7: (cfg["kv_heads"] * hd, H), 8: (cfg["kv_heads"] * hd, H),
              9: (H, cfg["heads"] * hd), 10: (I, H), 11: (I, H), 12: (H, I)}
    for layer in range(cfg["layers"]):
        yield 4, layer, norm(), None
        yield 5, layer, norm(), None
        for kind, (rows, cols) in shapes.items():
            q, sc = q8(rows, cols)
            yield kind, layer, q, sc


# Kernels of one graph-replayed decode token: the greedy pick from the previous head's keys with
# the embedding of the picked id; per layer the q/k/v GEMV, the split attention, the o, gate/up
# and down GEMVs; then the LM head (its RMSNorm inside, storing the greedy keys and advancing
# the position). Nothing runs between replays.
def decode_kernels_per_token(cfg):
    return 5 * cfg["layers"] + 2


def graph_node_floor_us(hip, nodes, reps=20):
    """Microseconds per node of a graph of `nodes` dependent minimal kernels (ResidualAdd over 64
    floats, each reading what the previous one wrote), replayed `reps` times after one untimed
    replay: the launch and memory round trip that a decode token's dependent kernels each pay
    before any of their own work."""
    buf = hip.DeviceArray.from_numpy(np.zeros(64, np.float32))

    def step(i):
        hip.check(hip.L.accel_hip_residual_add(buf.buffer, buf.buffer, 64))

    g = hip.graph(step, nodes)
    try:
        hip.check(hip.L.accel_hip_graph_launch(g, 1))
        ms = hip.time_graph([(g, reps)])
    finally:
        hip.L.accel_hip_graph_destroy(g)
    return ms * 1e3 / (nodes * reps)


class SmolModel:
    """The SmolLM2-135M-shape Llama of llama_q8_weights on the GPU (accel_llama_*) with a
    512-id random prompt; generate(new) runs a greedy generation and returns its wall time."""

    def __init__(self, hip, rng):
        from accelep_amd.capi import F32P, I8P, LlamaConfig

        self.L = L = hip.L
        self.h = L.accel_llama_create(C.byref(LlamaConfig(**SMOL)))
        if not self.h:
            raise RuntimeError(L.accel_llama_last_error().decode())
        try:
            for kind, layer, w, sc in llama_q8_weights(SMOL, rng):
                if sc is None:
                    rc = L.accel_llama_weight(self.h, kind, layer, w.ctypes.data_as(F32P), w.shape[0], 1)
                else:
                    rc = L.accel_llama_weight_q8(self.h, kind, layer, w.ctypes.data_as(I8P), sc.ctypes.data_as(F32P),
                                                 w.shape[0], w.shape[1])
                if rc != 0:
                    raise RuntimeError(L.accel_llama_last_error().decode())
        except BaseException:
            self.close()
            raise
        self.prompt = rng.integers(0, SMOL["vocab"], size=512).astype(np.int32)
        self.out = np.zeros(129, np.int32)

    def generate(self, new):
        from accelep_amd.capi import I32P

        count = C.c_int32()
        t0 = time.perf_counter()
        rc = self.L.accel_llama_generate(self.h, self.prompt.ctypes.data_as(I32P), self.prompt.size, new, -1, 0.0, 0,
                                         0, self.out.ctypes.data_as(I32P), C.byref(count))
        dt = time.perf_counter() - t0
        if rc != 0:
            raise RuntimeError(self.L.accel_llama_last_error().decode())
        return dt

    def close(self):
        if self.h:
            self.L.accel_llama_destroy(self.h)
            self.h = None


def bench_llama(hip, rng, reps=3):
    """SmolLM2-135M-shape Llama on the GPU (accel_llama_*): the int8 weights of
    llama_q8_weights, 512 random prompt ids, 128 greedy tokens. Prefill = generate with one
    new token; decode = the extra time of 128 more tokens. Best of `reps`."""
    cfg = SMOL
    model = SmolModel(hip, rng)
    generate = model.generate
    try:
        generate(129)  # warm-up: staging of the int8 weights, workspaces, the decode graph
        pre = min(generate(1) for _ in range(reps))
        full = min(generate(129) for _ in range(reps))
        decode = max(full - pre, 1e-9)
        kernels = decode_kernels_per_token(cfg)
        floor_us = graph_node_floor_us(hip, kernels)
        token_ms = decode / 128 * 1e3
        return {"prefill_ms": round(pre * 1e3, 2), "prefill_tok_s": round(512 / pre, 1),
                "decode_ms_per_token": round(token_ms, 4), "decode_tok_s": round(128 / decode, 1),
                "decode_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / LLAMA_DECODE_BYTES, 1),
                "decode_roofline_frac": round((128 / decode) / (HBM_PEAK_GBS * 1e9 / LLAMA_DECODE_BYTES), 4),
                "decode_kernels_per_token": kernels, "graph_node_floor_us": round(floor_us, 3),
                "decode_node_floor_ms": round(kernels * floor_us / 1e3, 4),
                "decode_node_floor_frac": round(kernels * floor_us / 1e3 / token_ms, 4),
                "config": "SmolLM2-135M shape (30 layers, hidden 576, 9/3 heads, inter 1536, vocab 49152), "
                          "linear weights and tied embedding/LM head N(0,0.02) quantized to int8 per output row, "
                          "norms N(1,0.1), 512 random prompt ids, 128 greedy tokens, wall clock, best of 3"}
    finally:
        model.close()


# Event slots the marked decode step records (the MarkSlot order of accelep_amd/csrc/llama.cc).
MARKS = ("start", "embedded", "layer", "qkv", "attention", "o", "gate_up", "down", "layers", "head_norm", "head",
         "advance", "sample_start", "sample_end", "node0", "node1")


def decode_marks(hip, layers, rng, reps=3):
    """Times the parts of one graph-replayed decode token from event nodes inside the captured
    step (ACCEL_LLAMA_DECODE_MARKS=<layer>; the last step of a 512-id prompt and 128 tokens,
    position 639): the greedy pick from the previous head's keys with the embedding (one kernel),
    the given layers' five kernels each, all 30 layers, and the LM head (one kernel: its norm,
    product, greedy keys and the position advance). The marks cover the graph from its first node;
    the host's launch of the graph between tokens is in the unmarked token only.
    Every mark is an event node of the graph, which takes about as long as a dependent kernel:
    each span holds the node that ends it, and two marks back to back at the start of the step
    time one node on its own (event_node_us). The unmarked token (decode_us_per_token_unmarked)
    is measured first. Best (smallest marked total) of `reps` generations per marked layer."""
    slot = {name: i for i, name in enumerate(MARKS)}

    def span(a, b):
        ms = hip.L.accel_hip_event_elapsed_ms(slot[a], slot[b])
        if ms < 0:
            raise RuntimeError(hip.L.accel_hip_last_error().decode())
        return ms * 1e3

    model = SmolModel(hip, rng)
    try:
        os.environ.pop("ACCEL_LLAMA_DECODE_MARKS", None)
        model.generate(129)
        plain = min(model.generate(129) - model.generate(1) for _ in range(reps)) / 128 * 1e6
        result = {"decode_us_per_token_unmarked": round(plain, 2), "layers": {}}
        for layer in layers:
            os.environ["ACCEL_LLAMA_DECODE_MARKS"] = str(layer)
            model.generate(128)  # captures the marked step
            best = None
            for _ in range(reps):
                model.generate(128)  # 128 tokens: the last one's sampler runs before the last graph replay
                parts = {
                    "graph start (3 event nodes)": span("node0", "start"),
                    "greedy pick and embedding (GreedyEmbedKernel)": span("start", "embedded"),
                    "layers 0-29": span("embedded", "layers"),
                    "LM head (RMSNorm, GEMV 576 x 49152, greedy keys, advance)": span("layers", "head"),
                }
                total = span("node0", "head")
                node = span("node0", "node1")
                layer_parts = {
                    "q/k/v GEMV (RMSNorm prologue)": span("layer", "qkv"),
                    "split attention (RoPE, KV append)": span("qkv", "attention"),
                    "o GEMV (attention combine, residual)": span("attention", "o"),
                    "gate/up GEMV (RMSNorm prologue)": span("o", "gate_up"),
                    "down GEMV (SiLU*up prologue, residual)": span("gate_up", "down"),
                }
                if best is None or total < best["token_us_marked"]:
                    best = {"token_us_marked": round(total, 2), "event_node_us": round(node, 2),
                            "parts_us": {k: round(v, 2) for k, v in parts.items()},
                            "layer_us": {k: round(v, 2) for k, v in layer_parts.items()}}
            result["layers"][str(layer)] = best
        os.environ.pop("ACCEL_LLAMA_DECODE_MARKS", None)
        return result
    finally:
        model.close()


def calibrate_traffic(hip):
    """One residual add over 16 Mi floats: a streaming kernel of known HBM traffic (128 MiB read,
    64 MiB written) whose FETCH_SIZE / WRITE_SIZE scale the GEMV's counters to bytes."""
    count = 16 << 20
    dst = hip.DeviceArray((count,))
    src = hip.DeviceArray((count,))
    hip.check(hip.L.accel_hip_residual_add(dst.buffer, src.buffer, count))
    hip.sync()
    dst.free()
    src.free()


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


class OneCore:
    """Pins the calling thread to one CPU of its current set for the CPU legs (the reference's
    SimDevice is single-threaded), in-process: sched_setaffinity on this thread, restored on
    exit. The GPU runtime's own threads keep their affinity."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        self.cpu = min(self.saved)
        os.sched_setaffinity(0, {self.cpu})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)


def _median_time(fn, runs):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


CPU_RUNS = 5  # every CPU leg: the median of this many timed runs after one warm-up


def cpu_baseline(rng, runs=CPU_RUNS):
    """The reference's MatMulQuantized (compiled AccelEP sources) on the M=1 headline workload,
    pinned to one core; median of `runs` after one warm-up call."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ctypes import make_plane, oracle, reference

    ref = reference()
    kind = "reference" if ref is not None else "port"
    impl = ref if ref is not None else oracle()
    q = rng.integers(-127, 128, size=K_DIM * N_DIM, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=N_DIM).astype(np.float32)
    a = rng.standard_normal((1, K_DIM)).astype(np.float32)
    plane, keep = make_plane(q, s, None, [K_DIM, N_DIM], 1)
    with OneCore() as core:
        impl.matmul_quantized(a, None, None, plane, 1, K_DIM, N_DIM)
        best = _median_time(lambda: impl.matmul_quantized(a, None, None, plane, 1, K_DIM, N_DIM), runs)
    return {
        "value": round(gemv_bytes(1) / best / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"full M=1 workload X[1,4096] @ int8 W[4096,14336] per-column scale, "
                   f"{'AccelEP MatMulQuantized (src/sim_device.cc:541-602) compiled -O2' if ref else 'oracle port'}, "
                   f"one thread pinned to CPU {core.cpu} ({cpu_model()}; host has {os.cpu_count()} logical CPUs), "
                   f"median of {runs} after a warm-up: {best:.2f} s/call"),
        "cpu_model": cpu_model(),
        "seconds_per_call": round(best, 3),
    }


def cpu_prefill_sample(rng, rows=64, cols=N_DIM // 8, runs=CPU_RUNS):
    """C4 on the reference path is hours, so it is timed on a block: X[rows,4096] @ int8
    W[4096,cols] (per-column scale) plus SimRmsNorm of the block's rows, pinned to one core, and
    extrapolated linearly to 2048 rows and 14336 columns (the reference blocks M by 64 and N by
    256, so its time is linear in both at these multiples)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ctypes import make_plane, reference

    ref = reference()
    if ref is None:
        return None
    q = rng.integers(-127, 128, size=K_DIM * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=cols).astype(np.float32)
    a = rng.standard_normal((rows, K_DIM)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    plane, keep = make_plane(q, s, None, [K_DIM, cols], 1)
    with OneCore() as core:
        def run():
            c = ref.matmul_quantized(a, None, None, plane, rows, K_DIM, cols)
            ref.rmsnorm(c, g, rows, cols, 1e-5, 0)
        run()
        t = _median_time(run, runs)
    scale = (2048 / rows) * (N_DIM / cols)
    total = t * scale
    return {"seconds_extrapolated": round(total, 1), "TFLOP/s": round(2 * 2048 * K_DIM * N_DIM / total / 1e12, 6),
            "cores": 1, "kind": "reference", "extrapolated": True,
            "sample": (f"AccelEP MatMulQuantized + SimRmsNorm on X[{rows},4096] @ int8 W[4096,{cols}], one thread "
                       f"pinned to CPU {core.cpu}, median of {runs} after a warm-up: {t:.2f} s, times {scale:.0f} for the full "
                       f"2048 x 4096 x 14336 workload (extrapolated)")}


def cpu_llama_sample(rng, prompt_ids=32, new=16, runs=CPU_RUNS):
    """C5 on the reference path (accel_llama_* of AccelEP's llama_model.cc through oracle/_ref)
    on a bounded sample: the SmolLM2-135M shape with the same weight generator (float weights
    fl(q*s), as the reference takes them), a `prompt_ids`-id prompt and `new` greedy tokens,
    pinned to one core. Prefill and decode are reported per token; the 512 + 128 workload's
    decode positions are longer, which adds the attention over ~600 cached rows (~1% of a
    token's 0.3 GFLOP of weights at this shape)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ctypes import F32P, I32P, LlamaConfig as RefConfig, reference

    ref = reference()
    if ref is None:
        return None
    L = ref.lib
    cfg = SMOL
    h = L.accel_llama_create(C.byref(RefConfig(**cfg)))
    if not h:
        return None
    try:
        for kind, layer, w, sc in llama_q8_weights(cfg, rng):
            f = w if sc is None else (w.astype(np.float32) * sc[:, None]).astype(np.float32)
            f = np.ascontiguousarray(f)
            rows, cols = (f.shape[0], 1) if f.ndim == 1 else f.shape
            if L.accel_llama_weight(h, kind, layer, f.ctypes.data_as(F32P), rows, cols) != 0:
                return None
        prompt = rng.integers(0, cfg["vocab"], size=prompt_ids).astype(np.int32)
        out = np.zeros(new + 1, np.int32)
        count = C.c_int32()

        def generate(k):
            t0 = time.perf_counter()
            rc = L.accel_llama_generate(h, prompt.ctypes.data_as(I32P), prompt.size, k, -1, 0.0, 0, 0,
                                        out.ctypes.data_as(I32P), C.byref(count))
            if rc != 0:
                raise RuntimeError(L.accel_llama_last_error().decode())
            return time.perf_counter() - t0

        with OneCore() as core:
            generate(1)
            pre = float(np.median([generate(1) for _ in range(runs)]))
            full = float(np.median([generate(new + 1) for _ in range(runs)]))
        decode = max(full - pre, 1e-9) / new
        return {"prefill_tok_s": round(prompt_ids / pre, 2), "decode_s_per_token": round(decode, 4),
                "decode_tok_s": round(1 / decode, 3), "cores": 1, "kind": "reference",
                "sample": (f"AccelEP LlamaModel Generate (src/llama_model.cc) compiled -O2, SmolLM2-135M shape, "
                           f"{prompt_ids}-id prompt ({pre:.2f} s) + {new} greedy tokens ({full - pre:.2f} s), "
                           f"one thread pinned to CPU {core.cpu}, medians of {runs} after a warm-up")}
    finally:
        L.accel_llama_destroy(h)


def mlp_inputs(rng):
    """The C2 MLP's operands: X[256,1024] ~ N(0,1); W1[1024,4096], b1, W2[4096,1024], b2 ~ N(0,0.02)."""
    m, d, h = MLP_SHAPE
    x = rng.standard_normal((m, d)).astype(np.float32)
    w1 = (rng.standard_normal((d, h)) * 0.02).astype(np.float32)
    b1 = (rng.standard_normal(h) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((h, d)) * 0.02).astype(np.float32)
    b2 = (rng.standard_normal(d) * 0.02).astype(np.float32)
    return x, w1, b1, w2, b2


def cpu_mlp(rng, runs=CPU_RUNS):
    """C2 on the reference path, the whole workload: SimDevice::MatMul (PackedMatMul,
    src/sim_device.cc:185-196,331-369), GemmEpilogue with bias and exact Gelu (:211-245), the
    second MatMul, GemmEpilogue with bias, and the residual as the runtime issues it
    (GemmEpilogue over m = 1, n = count with X as the bias, src/runtime.cc:332-344), through the
    compiled reference, pinned to one core; median of `runs` after one warm-up step."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ctypes import reference

    ref = reference()
    if ref is None:
        return None
    m, d, h = MLP_SHAPE
    x, w1, b1, w2, b2 = mlp_inputs(rng)

    def step():
        hid = ref.gemm_epilogue(ref.device_matmul(x, w1), 1.0, b1, [h], 1.0, 2)
        y = ref.gemm_epilogue(ref.device_matmul(hid, w2), 1.0, b2, [d], 1.0, 0)
        return ref.gemm_epilogue(y.reshape(1, m * d), 1.0, x.reshape(-1), [m * d], 1.0, 0)

    with OneCore() as core:
        step()
        t = _median_time(step, runs)
    flops = 2 * m * d * h * 2
    return {"seconds_per_step": round(t, 3), "TFLOP/s": round(flops / t / 1e12, 6), "cores": 1, "kind": "reference",
            "sample": (f"the whole C2 step through AccelEP SimDevice (src/sim_device.cc MatMul + GemmEpilogue, "
                       f"residual as src/runtime.cc:332-344 issues it) compiled -O2, one thread pinned to CPU "
                       f"{core.cpu}, median of {runs} after a warm-up: {t:.2f} s/step")}


def bench_c1(hip, steps, warmup, rng):
    """C1: X fp32[4,576] @ DequantizeLinear(int8 W[576,1536], per-column scale, zero point 0) as
    accel::MatMulQuantized, one call a step. Returns (ms_per_step, GB/s of algorithmic bytes)."""
    m, k, n = C1_SHAPE
    q = hip.DeviceArray.from_numpy(rng.integers(-127, 128, size=k * n, dtype=np.int8))
    s = hip.DeviceArray.from_numpy(rng.uniform(1e-3, 1e-2, size=n).astype(np.float32))
    plane = hip.quant_plane(q, s, None, [k, n], 1)
    x = hip.DeviceArray.from_numpy(rng.standard_normal((m, k)).astype(np.float32))
    out = hip.DeviceArray((m, n))

    def step(i):
        hip.check(hip.L.accel_hip_matmul_quantized(x.ptr, None, None, C.byref(plane), out.ptr, m, k, n))

    ms = timed_steps(hip, step, steps, warmup)
    per = ms / steps
    return per, gemv_bytes(m, k, n) / (per * 1e-3) / 1e9


def cpu_c1(rng, runs=CPU_RUNS):
    """C1 on the reference path: AccelEP's MatMulQuantized (src/sim_device.cc:541-602) on
    X[4,576] @ int8 W[576,1536] with a per-column scale, pinned to one core; median of `runs`
    after one warm-up call."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ctypes import make_plane, reference

    ref = reference()
    if ref is None:
        return None
    m, k, n = C1_SHAPE
    q = rng.integers(-127, 128, size=k * n, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    plane, keep = make_plane(q, s, None, [k, n], 1)
    with OneCore() as core:
        ref.matmul_quantized(a, None, None, plane, m, k, n)
        t = _median_time(lambda: ref.matmul_quantized(a, None, None, plane, m, k, n), runs)
    return {"seconds_per_call": round(t, 5), "GB/s": round(gemv_bytes(m, k, n) / t / 1e9, 5), "cores": 1,
            "kind": "reference",
            "sample": (f"the whole C1 call, AccelEP MatMulQuantized compiled -O2, one thread pinned to CPU {core.cpu}, "
                       f"median of {runs} after a warm-up: {t * 1e3:.1f} ms/call")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--only-llama", action="store_true", help="run only the Llama decode leg (for profiling)")
    ap.add_argument("--only-gemm", action="store_true",
                    help="run only the MFMA legs (int8 prefill GEMM + RMSNorm, fp32 MLP), for profiling")
    ap.add_argument("--only-sweep", action="store_true",
                    help="run only the M = 4 and M = 16 int8 GEMVs of the decode sweep (for profiling)")
    ap.add_argument("--no-graph", action="store_true", help="launch each step directly instead of from HIP graphs")
    ap.add_argument("--decode-marks", default=None, metavar="LAYERS",
                    help="time the parts of a graph-replayed decode token (event nodes around the given layers' "
                         "kernels, comma separated) and print them as one JSON line")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run one residual add of known traffic (for profiler counter scaling)")
    args = ap.parse_args()
    global GRAPHS
    GRAPHS = not args.no_graph
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the hot path runs on a single MI355X and there is no "
              f"multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("steps must be >= 1 and warmup >= 0")

    rng = np.random.default_rng(20251201)
    hip = Hip()
    log(f"device {hip.arch}")

    if args.decode_marks is not None:
        layers = [int(v) for v in args.decode_marks.split(",") if v != ""]
        print(json.dumps({"decode_marks": decode_marks(hip, layers, np.random.default_rng(11))}), flush=True)
        return
    if args.only_llama:
        llama = bench_llama(hip, np.random.default_rng(11))
        print(json.dumps({"llama_decode": llama}), flush=True)
        return
    if args.only_gemm:
        out = {}
        for name, leg in (("prefill_int8_rmsnorm", bench_prefill), ("mlp_fp32", bench_mlp)):
            per, tf = leg(hip, args.steps, args.warmup, rng)
            out[name] = {"ms_per_step": round(per, 4), "TFLOP/s": round(tf, 2),
                         "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
            if name.startswith("prefill"):
                out[name]["mfma_frac"] = None
                out[name]["vs_fp32_mfma_peak"] = round(tf / FP32_MFMA_PEAK_TFLOPS, 4)
                out[name]["bf16x3_roofline_frac"] = round(tf / BF16X3_PEAK_TFLOPS, 4)
            log(f"{name}: {per:.4f} ms/step, {tf:.1f} TFLOP/s")
        print(json.dumps(out), flush=True)
        return
    if args.only_sweep:
        if args.calibrate:
            calibrate_traffic(hip)
        out = {}
        for m in (4, 16):
            per, gbs = bench_gemv(hip, m, args.steps, args.warmup, COPIES, rng)
            out[f"gemv_m{m}"] = {"us_per_step": round(per * 1e3, 3), "GB/s": round(gbs, 1),
                                 "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            log(f"gemv M={m}: {per * 1e3:.2f} us/step, {gbs:.1f} GB/s")
        print(json.dumps(out), flush=True)
        return
    if args.calibrate:
        calibrate_traffic(hip)
    per1, gbs1 = bench_gemv(hip, 1, args.steps, args.warmup, COPIES, rng)
    log(f"gemv M=1 (HBM, {COPIES} copies): {per1 * 1e3:.2f} us/step, {gbs1:.1f} GB/s")
    secondary = {}
    if not args.only_headline:
        # The secondary GEMV legs time at least 400 steps (one graph; a few ms), so their lines
        # carry the steady per-step time rather than one graph launch spread over a few steps.
        steps_g = max(400, args.steps)
        for m in (4, 16):
            per, gbs = bench_gemv(hip, m, steps_g, args.warmup, COPIES, rng)
            flops = 2 * m * K_DIM * N_DIM
            secondary[f"gemv_m{m}"] = {"us_per_step": round(per * 1e3, 3), "GB/s": round(gbs, 1),
                                       "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                       "TFLOP/s": round(flops / (per * 1e-3) / 1e12, 2), "steps": steps_g}
            log(f"gemv M={m}: {per * 1e3:.2f} us/step, {gbs:.1f} GB/s")
        per, gbs = bench_c1(hip, steps_g, args.warmup, rng)
        secondary["c1_dequant_matmul"] = {"us_per_step": round(per * 1e3, 3), "GB/s": round(gbs, 1), "steps": steps_g,
                                          "config": "X fp32[4,576] @ int8 W[576,1536], per-column scale (C1)",
                                          "note": "latency-bound: 0.92 MB, one launch"}
        log(f"c1 4x576x1536: {per * 1e3:.2f} us/step")
        per, gbs = bench_gemv(hip, 1, steps_g, args.warmup, 1, rng)
        secondary["gemv_m1_cache_warm"] = {"us_per_step": round(per * 1e3, 3), "GB/s": round(gbs, 1), "steps": steps_g,
                                           "note": "one weight copy, L2/MALL may serve it; not HBM-honest"}
        # The GEMM legs time at least 20 launches after at least 5 untimed ones, whatever
        # --steps is: a leg that follows the memory-bound GEMV legs runs its first launches
        # while the clocks settle.
        steps2 = max(20, args.steps // 4)
        per, tf = bench_mlp(hip, steps2, max(5, args.warmup // 4), rng)
        secondary["mlp_fp32"] = {"ms_per_step": round(per, 4), "TFLOP/s": round(tf, 2),
                                 "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "steps": steps2,
                                 "config": "X[256,1024] Gemm1024x4096+bias+gelu, Gemm4096x1024+bias+residual"}
        log(f"mlp fp32: {per:.3f} ms/step, {tf:.1f} TFLOP/s")
        steps4 = max(20, args.steps // 20)
        per, tf = bench_prefill(hip, steps4, max(5, args.warmup // 20), rng)
        secondary["prefill_int8_rmsnorm"] = {
            "ms_per_step": round(per, 4), "TFLOP/s": round(tf, 2),
            "vs_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "bf16x3_roofline_frac": round(tf / BF16X3_PEAK_TFLOPS, 4),
            "kernel": "GemmQ8Bf16WideKernel (accelep_amd/csrc/gemm_q8_bf16.hip): exact fp32 products as 3 bf16 MFMA passes, roofline 833 TFLOP/s",
            "steps": steps4, "config": "X[2048,4096] @ int8 W[4096,14336] + RMSNorm(eps 1e-5)"}
        log(f"prefill int8+rms: {per:.3f} ms/step, {tf:.1f} TFLOP/s")
        llama = bench_llama(hip, np.random.default_rng(11))
        secondary["llama_decode"] = llama
        log(f"llama: prefill {llama['prefill_ms']} ms ({llama['prefill_tok_s']} tok/s), "
            f"decode {llama['decode_ms_per_token']} ms/token ({llama['decode_tok_s']} tok/s)")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (reference MatMulQuantized, 1 pinned thread) ...")
        cpu = cpu_baseline(np.random.default_rng(7))
        log(f"cpu baseline: {cpu['value']} GB/s ({cpu['seconds_per_call']} s/call)")
        if not args.only_headline:
            pf = cpu_prefill_sample(np.random.default_rng(8))
            if pf is not None and "prefill_int8_rmsnorm" in secondary:
                secondary["prefill_int8_rmsnorm"]["cpu_reference"] = pf
                log(f"cpu prefill (extrapolated): {pf['seconds_extrapolated']} s")
            c1 = cpu_c1(np.random.default_rng(10))
            if c1 is not None and "c1_dequant_matmul" in secondary:
                secondary["c1_dequant_matmul"]["cpu_reference"] = c1
                log(f"cpu c1: {c1['seconds_per_call'] * 1e3:.1f} ms/call")
            mlp = cpu_mlp(np.random.default_rng(12))
            if mlp is not None and "mlp_fp32" in secondary:
                secondary["mlp_fp32"]["cpu_reference"] = mlp
                log(f"cpu mlp: {mlp['seconds_per_step']} s/step")
            ll = cpu_llama_sample(np.random.default_rng(9))
            if ll is not None and "llama_decode" in secondary:
                secondary["llama_decode"]["cpu_reference"] = ll
                log(f"cpu llama: decode {ll['decode_s_per_token']} s/token, prefill {ll['prefill_tok_s']} tok/s")

    line = {
        "metric": METRIC,
        "value": round(gbs1, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per1, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "int8-weight decode GEMV: X fp32[1,4096] @ W int8[4096,14336], per-column fp32 scale "
                        "(accel::MatMulQuantized), 8 weight copies rotated to defeat the 256 MB MALL",
            "weights": "int8 uniform [-127,127], scale uniform [1e-3,1e-2], X ~ N(0,1)",
            "parallelism": "1 GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs1, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs1 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": str(TRAFFIC_PROFILE.relative_to(ROOT)),
            "kernel": "GemvM1Kernel<8,false,true,0,false> (accelep_amd/csrc/gemv_q8.hip)",
            "algorithmic_bytes_per_launch": gemv_bytes(1),
            "avg_launch_us_event_timed": round(per1 * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
