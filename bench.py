#!/usr/bin/env python3
"""Benchmark of the Q4_0 ring decode-attention path on one MI355X.

Default workload: one step = decode attention of 64
sessions through 32 layers (32 launches), 32 heads x head_dim 128, full
W=512 windows at per-session positions in [512, 4096), K/V ~N(0,1) with each
element scaled x8 with probability 1%, quantized to Q4_0 by the library's
own write kernel.  The ring (4.83 GB) is resident in HBM before timing
starts.  Every input is the configuration's seeded stream (splitmix64 +
Box-Muller, seeds 0xB0A00001..5; layouts in fill_ring, run_decode and each
leg), generated on the GPU by libbmo_synth.so, bit for bit the stream the
CPU restates, so any part of it can be regenerated from the seed.

value = algorithmic bytes per step / step time, where the algorithmic bytes
of one (session, layer) are the full window's Q4_0 K+V bytes
(W*H*2*(D/32)*18) plus q and out in fp32 (2*H*D*4): 2,392,064 B, so
4,898,947,072 B per step.

The step (32 launches, one per layer) is captured in a HIP graph before the
ring is filled; after the fill, one eager step, --warmup untimed replays and
exactly --steps timed replays between two synchronizations, timed by a HIP
event pair on the replay stream.  The roofline entry divides one launch's
algorithmic bytes by the mean launch duration from that region (step time /
32, kernel gaps included).

Also reported: BASELINE config 4 (256 sessions, fused append + decode, timed
the same way, with its own roofline entry), B=1 latency (one layer, 32 heads, W=512,
write head at position 700; fused append+decode as the reference kernel does,
and decode alone), the depformer frame, and the CPU
baseline timed on this host on a bounded sample of the same ring: a
restatement of ggml's CPU flash attention over Q4_0 (the reference's lazy
backend), and the reference's own scalar CPU loop restated in fp32.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg3|cfg4]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "Q4_0 KV GB/s + % of 8 TB/s HBM at B=64 W=512 32L; µs/layer at B=1"
HBM_PEAK_GBS = 8000.0


def unit_bytes(H, D, W):
    """Algorithmic bytes of one (session, layer) decode."""
    return W * H * 2 * (D // 32) * 18 + 2 * H * D * 4


def fused_extra_bytes(H, D):
    """New K/V fp32 rows read plus their Q4_0 blocks written, per (session, layer)."""
    return 2 * H * D * 4 + 2 * H * (D // 32) * 18


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def read_traffic(config):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the
    copy-kernel calibration), or None when there is none for this workload."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"decode_{config}_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def fill_ring(torch, ring, L, S, H, D, W, pos_end, seed, outliers=True):
    """Writes each session's window of positions pos_end[s] - W + 1 ..
    pos_end[s] in every layer.  K of (layer l, session s, window slot j
    (position pos_end[s] - W + 1 + j), head h, dim d) is element
    (((l S + s) W + j) H + h) D + d of the seeded stream `seed` (x8 with
    probability 1% when `outliers`), V the same element of stream seed + 1;
    generated on the GPU by libbmo_synth.so, bit for bit the CPU's
    restatement."""
    from bmo_jetson_amd.synth import fill_normal

    stream = torch.cuda.current_stream()
    k = torch.empty((S, W, H, D), device="cuda")
    v = torch.empty((S, W, H, D), device="cuda")
    for layer in range(L):
        off = layer * S * W * H * D
        fill_normal(k, seed, off, outliers, stream=stream)
        fill_normal(v, seed + 1, off, outliers, stream=stream)
        for s in range(S):
            ring.write(layer, s, int(pos_end[s]) - W + 1, k[s], v[s], stream=stream)
    torch.cuda.synchronize()
    del k, v


def synth(torch, shape, seed, offset=0):
    """A device tensor of `shape` holding elements offset.. of stream seed."""
    from bmo_jetson_amd.synth import fill_normal

    t = torch.empty(shape, device="cuda")
    fill_normal(t, seed, offset, stream=torch.cuda.current_stream())
    return t


def capture_graph(torch, launch):
    """Captures launch(stream) into a HIP graph on a side stream."""
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            launch(torch.cuda.current_stream())
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return graph


def time_steps(torch, launch_layer, n_layers, steps, warmup, prepare=None):
    """Captures one step (n_layers launches, one per layer, as the model runs
    them) into a HIP graph, then runs prepare() (the inputs' generation and
    the ring fill: capture needs only the buffers' addresses, so the GPU's
    heavy setup work ends right before the timed part instead of an idle
    spell of capturing, after which the first milliseconds of work ran about
    2% slower), one eager step, `warmup` untimed graph replays, and exactly
    `steps` replays between two torch.cuda.synchronize() calls, timed with a
    HIP event pair recorded on the replay stream.  Returns ms per step; the
    mean launch duration is that over n_layers (it includes the small gaps
    between the graph's kernels, so it is an upper bound on the kernel time).
    Then `steps` more replays, each between its own event pair, give the
    per-step distribution (median, min, max), outside the timed region."""
    def whole_step(st):
        for layer in range(n_layers):
            launch_layer(layer, st)

    graph = capture_graph(torch, whole_step)
    if prepare is not None:
        prepare()
    stream = torch.cuda.current_stream()
    whole_step(stream)
    for _ in range(warmup):
        graph.replay()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(steps):
        graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        graph.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    del graph
    return ms, per_step


def graph_us_per_call(torch, call, calls_per_graph, reps=20, warm_ms=100.0):
    """Microseconds per call from HIP-graph replays of calls_per_graph calls:
    `reps` replays timed by one event pair, after untimed replays worth at
    least warm_ms of GPU time.  The clocks rise over the first tens of
    milliseconds of sustained work: replays of ten cfg5 prefill calls measured
    92 us per call at first, 80 after 20 replays and 74-76 from about 60 on."""
    graph = capture_graph(torch, lambda st: [call(st) for _ in range(calls_per_graph)])
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    for _ in range(max(1, int(warm_ms / max(e0.elapsed_time(e1), 1e-3)))):
        graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1000.0 / (reps * calls_per_graph)


def bench_b1(torch, iters=200):
    """BASELINE config 1 at B=1: per-launch time of one layer, from a HIP graph
    of `iters` back-to-back launches (what a captured decode step replays) and
    from an eager loop (Python launch cost included)."""
    from bmo_jetson_amd import KVRing

    H, D, W, P, seed = 32, 128, 512, 700, 0xB0A00001
    ring = KVRing(1, 1, H, D, W)
    # the ring holds positions 189..700 (streams seed, seed + 1); q, k, v are
    # streams seed + 2, + 3, + 4 (the fused call appends k, v at 700 again)
    fill_ring(torch, ring, 1, 1, H, D, W, [P], seed, outliers=False)
    stream = torch.cuda.current_stream()
    pos = torch.tensor([P], dtype=torch.int32, device="cuda")
    q, k, v = (synth(torch, (H * D,), seed + i) for i in (2, 3, 4))
    out = torch.empty(H * D, device="cuda")
    res = {}
    calls = {
        "fused": lambda st: ring.append_decode(0, pos, q, k, v, out, H, stream=st),
        "fused_rope": lambda st: ring.append_decode(0, pos, q, k, v, out, H, stream=st,
                                                    rope_theta=10000.0),
        "decode": lambda st: ring.decode(0, pos, q, out, H, stream=st),
    }
    for name, fn in calls.items():
        for _ in range(20):
            fn(stream)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn(stream)
        e1.record()
        torch.cuda.synchronize()
        eager_us = e0.elapsed_time(e1) * 1000.0 / iters
        res[name] = {"graph_us": round(graph_us_per_call(torch, fn, iters), 3),
                     "eager_us": round(eager_us, 3)}
    ring.close()
    b = unit_bytes(H, D, W)
    cold = bench_b1_cold(torch)
    return {
        "workload": "cfg1: S=1 L=1 H=32 D=128 W=512 pos=700",
        "us_per_layer_cold_32L_fused_graph": cold["fused"],
        "us_per_layer_cold_32L_decode_graph": cold["decode"],
        "cold_note": cold["note"],
        "graph_launch_floor_us": graph_launch_floor_us(torch),
        "us_per_layer_fused_graph": res["fused"]["graph_us"],
        "us_per_layer_fused_eager": res["fused"]["eager_us"],
        "us_per_layer_fused_rope_graph": res["fused_rope"]["graph_us"],
        "us_per_layer_decode_graph": res["decode"]["graph_us"],
        "us_per_layer_decode_eager": res["decode"]["eager_us"],
        "decode_GBps_graph": round(b / (res["decode"]["graph_us"] * 1e-6) / 1e9, 1),
        "target_us": 10.0,
    }


def graph_launch_floor_us(torch, calls=200):
    """Microseconds per launch of a graph of `calls` launches of a kernel with
    no work to speak of (the library's position advance on one int): the
    floor under any per-call latency measured from a graph on this box."""
    from bmo_jetson_amd import positions_advance
    dummy = torch.zeros(1, dtype=torch.int32, device="cuda")
    return round(graph_us_per_call(torch, lambda st: positions_advance(dummy, 1, 0, stream=st),
                                   calls), 3)


def bench_b1_cold(torch, replicas=8):
    """BASELINE config 1 as a model step runs it: 32 layers (one launch each,
    32 distinct layer windows) at B=1, with the ring held `replicas` times
    (612 MB) and consecutive steps on consecutive replicas, so that each
    layer's 2.4 MB window has left the 256 MB last-level cache before it is
    read again (in the model, the weights streamed between layers evict it).
    Microseconds per launch from HIP-graph replays of `replicas` steps."""
    from bmo_jetson_amd import KVRing

    H, D, W, P, L, seed = 32, 128, 512, 700, 32, 0xB0A00011
    ring = KVRing(L, replicas, H, D, W)
    fill_ring(torch, ring, L, replicas, H, D, W, [P] * replicas, seed, outliers=False)
    q, k, v = (synth(torch, (L, H * D), seed + i) for i in (2, 3, 4))
    out = torch.empty((L, H * D), device="cuda")
    pos = torch.tensor([P], dtype=torch.int32, device="cuda")
    sids = [torch.tensor([r], dtype=torch.int32, device="cuda") for r in range(replicas)]
    res = {}
    for name in ("fused", "decode"):
        def steps(st, name=name):
            for r in range(replicas):
                for layer in range(L):
                    if name == "fused":
                        ring.append_decode(layer, pos, q[layer], k[layer], v[layer], out[layer], H,
                                           session_ids=sids[r], stream=st)
                    else:
                        ring.decode(layer, pos, q[layer], out[layer], H, session_ids=sids[r],
                                    stream=st)
        steps(torch.cuda.current_stream())
        torch.cuda.synchronize()
        res[name] = round(graph_us_per_call(torch, steps, 1, reps=10) / (replicas * L), 3)
    ring.close()
    res["note"] = (f"{replicas} ring replicas x {L} layers ({replicas * L * unit_bytes(H, D, W) / 1e6:.0f}"
                   " MB), one replica per step: every window is read from HBM")
    return res


def bench_depformer(torch, frames=20):
    """one depformer frame = the ring reset that
    bmo_forward_depth_cascade does first (src/bmo_api.cpp:682), then 8
    codebook steps x 6 layers of fused append+decode (16 heads x head_dim 64,
    8-slot ring, step s attends to steps 0..s), replayed from a HIP graph."""
    from bmo_jetson_amd import KVRing

    L, H, D, W, STEPS, seed = 6, 16, 64, 8, 8, 0xB0A00002
    ring = KVRing(L, 1, H, D, W)
    # q, k, v of (step, layer, head, dim): streams seed, seed + 1, seed + 2
    q, k, v = (synth(torch, (STEPS, L, H * D), seed + i) for i in (0, 1, 2))
    out = torch.empty((STEPS, L, H * D), device="cuda")
    pos = [torch.tensor([s], dtype=torch.int32, device="cuda") for s in range(STEPS)]

    def frame(st):
        ring.reset(0, stream=st)
        for s in range(STEPS):
            for layer in range(L):
                ring.append_decode(layer, pos[s], q[s, layer], k[s, layer], v[s, layer],
                                   out[s, layer], H, stream=st)

    stream = torch.cuda.current_stream()
    for _ in range(3):
        frame(stream)
    torch.cuda.synchronize()
    us_frame = graph_us_per_call(torch, frame, frames)
    ring.close()
    # KV read by step s: (s+1) slots x H x 2 x (D/32) x 18 B; q, out fp32; the
    # appended rows read as fp32 and written as Q4_0.
    frame_bytes = sum((s + 1) * H * 2 * (D // 32) * 18 for s in range(STEPS)) * L \
        + STEPS * L * (2 * H * D * 4 + fused_extra_bytes(H, D))
    return {
        "workload": "cfg2: depformer L=6 H=16 D=64 W=8, 8 steps per frame, reset + fused "
                    "append+decode",
        "graph_launch_floor_us": graph_launch_floor_us(torch),
        "us_per_frame_graph": round(us_frame, 3),
        "us_per_call_graph": round(us_frame / (STEPS * L), 3),
        "calls_per_frame": STEPS * L,
        "bytes_per_frame": frame_bytes,
    }


def bench_prefill(torch, reps=10):
    """chunked prefill of S=16 sessions x C=256 tokens into
    a W=512 ring, 32 heads x head_dim 128, bf16 q/k/v ~N(0,1), one layer per
    call (stage + attention + commit), with the ring history full (p0 = 1024)
    and empty (p0 = 0).  Timed as HIP-graph replays."""
    from bmo_jetson_amd import KVRing

    S, C, W, H, D, seed = 16, 256, 512, 32, 128, 0xB0A00005
    res = {"workload": "cfg5: S=16 sessions x C=256 tokens, W=512, H=32, D=128, bf16 q/k/v, "
                       "causal + window mask; one layer per call"}
    for name, p0 in (("full", 1024), ("empty", 0)):
        ring = KVRing(1, S, H, D, W)
        if p0:  # history: positions p0 - W .. p0 - 1 (streams seed, seed + 1)
            fill_ring(torch, ring, 1, S, H, D, W, [p0 - 1] * S, seed, outliers=False)
        # the chunk's q, k, v (session, token, head, dim): streams seed + 2,
        # + 3, + 4 rounded to bf16 (nearest even)
        q, k, v = (synth(torch, (S, C, H, D), seed + i).to(torch.bfloat16) for i in (2, 3, 4))
        out = torch.empty((S, C, H, D), device="cuda")
        pos0 = torch.full((S,), p0, dtype=torch.int32, device="cuda")
        call = lambda st: ring.prefill(0, pos0, q, k, v, out, H, n_tok=C, stream=st)
        for _ in range(3):
            call(torch.cuda.current_stream())
        torch.cuda.synchronize()
        us = graph_us_per_call(torch, call, reps)
        ring.close()
        keys = sum(min(p0 + i + 1, W) for i in range(C))  # keys seen per (session, head)
        flops = 4 * D * keys * H * S
        # algorithmic bytes: bf16 q/k/v in, fp32 out, the old window read
        # once (Q4_0), the chunk's Q4_0 blocks written once
        old = min(p0, W - 1) * H * 2 * (D // 32) * 18 * S
        qb = S * C * H * D * 2
        blocks = S * C * H * 2 * (D // 32) * 18
        bytes_ = 3 * qb + S * C * H * D * 4 + old + blocks
        res[name] = {"p0": p0, "us_per_layer": round(us, 2), "gflop": round(flops / 1e9, 2),
                     "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                     "mfma_frac_of_2500": round(flops / (us * 1e-6) / 2.5e15, 4),
                     "bytes": bytes_, "GBps": round(bytes_ / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(bytes_ / (us * 1e-6) / 8e12, 4)}
    return res


def prefill_phases(torch, reps=10):
    """Phase timings of the cfg5 prefill kernel from the diagnostic library
    libbmo_attn_phases.so (its prefill kernel records s_memtime at each
    phase boundary of every wave; see prefill.hip).  Per case the calls run
    as the prefill leg times them (graph replays after warm-up), and the last
    call's stamps are read; the summary gives medians over the
    workgroups of each round of 256 (the rounds cannot overlap: one workgroup
    fills a CU) and over the barrier periods of the tile loop, in us, and the
    instrumented calls' duration.  Run in its own process: it loads the
    diagnostic library in place of libbmo_attn.so."""
    import ctypes
    from bmo_jetson_amd import KVRing, _lib

    lib = ctypes.CDLL(_lib.LIB_PATH)
    lib.bmo_prefill_phase_stamps.restype = ctypes.c_int
    lib.bmo_prefill_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    S, C, W, H, D, seed = 16, 256, 512, 32, 128, 0xB0A00005
    NWG, NW, REC = 512, 16, 128
    res = {"workload": "cfg5, one layer per call; medians over workgroups (per round) and periods",
           "library": os.path.basename(_lib.LIB_PATH)}
    for name, p0 in (("full", 1024), ("empty", 0)):
        ring = KVRing(1, S, H, D, W)
        if p0:
            fill_ring(torch, ring, 1, S, H, D, W, [p0 - 1] * S, seed, outliers=False)
        q, k, v = (synth(torch, (S, C, H, D), seed + i).to(torch.bfloat16) for i in (2, 3, 4))
        out = torch.empty((S, C, H, D), device="cuda")
        pos0 = torch.full((S,), p0, dtype=torch.int32, device="cuda")
        call = lambda st: ring.prefill(0, pos0, q, k, v, out, H, n_tok=C, stream=st)
        for _ in range(3):
            call(torch.cuda.current_stream())
        torch.cuda.synchronize()
        # graph replays as in the prefill leg (warm clocks); the stamps are
        # those of the last call replayed
        call_us = graph_us_per_call(torch, call, reps)
        a = np.zeros(NWG * NW * REC, dtype=np.uint64)
        assert lib.bmo_prefill_phase_stamps(a.ctypes.data, a.nbytes) == 0
        ring.close()
        a = a.astype(np.int64).reshape(NWG, NW, REC)
        ticks_per_us = np.median((a[:, :, 6] - a[:, :, 1]) / ((a[:, :, 7] - a[:, :, 0]) / 100.0))
        us = lambda x: x / ticks_per_us
        start = (a[:, :, 0].min(1) - a[:, :, 0].min()) / 100.0  # real-time clock: 100 MHz
        first = start < np.median(start)
        case = {"p0": p0, "call_us": round(call_us, 2),
                "kernel_span_us": round((a[:, :, 7].max() - a[:, :, 0].min()) / 100.0, 2),
                "shader_clock_GHz": round(ticks_per_us / 1000.0, 3)}
        for rname, sel in (("round1", first), ("round2", ~first)):
            b = a[sel]
            case[rname] = {
                "workgroups": int(sel.sum()),
                "start_us": round(float(np.median(start[sel])), 2),
                "query_rows_converted_us": round(float(np.median(us(b[:, :, 2] - b[:, :, 1]))), 2),
                "chunk_quantized_us": round(float(np.median(us(b[:, :, 3] - b[:, :, 2]))), 2),
                "loop_us": round(float(np.median(us(b[:, :, 5] - b[:, :, 4]))), 2),
                "epilogue_us": round(float(np.median(us(b[:, :, 6] - b[:, :, 5]))), 2),
            }
        n = int(np.median(a[:, :, 8]))
        P = min(n, REC - 16) // 4
        per = a[:, :, 16:16 + 4 * P].reshape(NWG, NW, P, 4)
        A, B, Cd, Dd = (per[..., i] for i in range(4))
        nxt = np.concatenate([A[:, :, 1:], a[:, :, 5:6]], axis=2)
        loaders = slice(0, NW // 2)
        others = slice(NW // 2, NW)
        med = lambda x: round(float(np.median(x)), 3)
        case["periods"] = P
        case["period_us"] = med(us(nxt[:, 0] - A[:, 0]))
        case["loading_waves"] = {"dequantize_us": med(us(B - A)[:, loaders]),
                                 "barrier_wait_us": med(us(Cd - B)[:, loaders]),
                                 "multiply_us": med(us(nxt - Dd)[:, loaders])}
        case["other_waves"] = {"barrier_wait_us": med(us(Cd - B)[:, others]),
                               "ring_writes_us": med(us(Dd - Cd)[:, others]),
                               "multiply_us": med(us(nxt - Dd)[:, others])}
        mult = us(nxt - Dd).sum(2)  # per wave, over the loop
        case["multiply_total_us_by_wave_age"] = [round(float(np.median(mult[:, 4 * g:4 * g + 4])), 2)
                                                 for g in range(4)]
        case["multiply_total_us_by_wave_age_note"] = ("waves 4g .. 4g + 3: the (g+1)-th wave of each SIMD "
                                                      "(wave w runs on SIMD w mod 4), oldest first")
        res[name] = case
    return res


def bench_gemv(torch, reps=50):
    """The Q4_0 x Q8_1 GEMV of the projections around attention, at the
    reference's bench shapes (src/bmo_kernel_bench.cu:387-389) and the output
    projection, x = 0.5 as in the reference bench.  Per call from HIP-graph
    replays; GB/s counts the Q4_0 weight bytes (18 per 32 elements)."""
    import ctypes
    from bmo_jetson_amd import _lib
    res = {}
    L = _lib.lib()
    for name, rows, cols in (("qkv_12288x4096", 12288, 4096), ("out_4096x4096", 4096, 4096),
                             ("gate_in_11264x4096", 11264, 4096), ("gate_out_4096x5632", 4096, 5632)):
        nbytes = rows * cols // 32 * 18
        # enough weight copies that one graph's calls stream > 600 MB, so the
        # 256 MB last-level cache cannot serve them
        n_copies = -(-600_000_000 // nbytes)
        w = torch.randint(0, 256, (n_copies, nbytes), dtype=torch.uint8, device="cuda")
        # scales: finite fp16 values in [0.001, 0.06) in every block's first two bytes
        wv = w.view(-1, 18)
        wv[:, 0:2] = torch.empty(wv.shape[0], dtype=torch.float16, device="cuda").uniform_(
            0.001, 0.06).view(torch.uint8).view(-1, 2)
        x = torch.full((cols,), 0.5, device="cuda")
        y = torch.empty(rows, device="cuda")
        state = {"i": 0}

        def call(st, w=w, x=x, y=y, rows=rows, cols=cols, n_copies=n_copies, state=state):
            wp = w[state["i"] % n_copies]
            state["i"] += 1
            rc = L.bmo_launch_gemv_q4_0_q8_1(ctypes.c_void_p(wp.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                             ctypes.c_void_p(y.data_ptr()), rows, cols, None,
                                             ctypes.c_void_p(st.cuda_stream))
            assert rc == 0

        for _ in range(5):
            call(torch.cuda.current_stream())
        torch.cuda.synchronize()
        us = graph_us_per_call(torch, call, max(reps, n_copies))
        # the read probe over the same weight copies: one launch's ceiling
        ceil = read_ceiling(torch, [w[i].data_ptr() for i in range(n_copies)], nbytes, reps)
        del w
        res[name] = {"us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(nbytes / (us * 1e-6) / 8e12, 4), "weight_bytes": nbytes,
                     "read_probe_us": ceil["us_per_launch"]}
    return res


def read_ceiling(torch, ptrs, nbytes, reps=20):
    """The read probe of libbmo_synth.so (one 16-byte nontemporal load per
    thread, the fastest single-pass read pattern measured) over the buffers
    at device addresses ptrs, nbytes each, one launch per buffer in turn,
    timed like a kernel leg (graph replays): the ceiling for one launch that
    reads those bytes once."""
    from bmo_jetson_amd.synth import read_probe

    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    state = {"i": 0}

    def call(st):
        read_probe(ptrs[state["i"] % len(ptrs)], nbytes, sink, stream=st)
        state["i"] += 1

    us = graph_us_per_call(torch, call, max(reps, len(ptrs)))
    return {"bytes_per_launch": nbytes, "us_per_launch": round(us, 3),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 8e12, 4)}


def run_decode(torch, config, steps, warmup, sessions=None):
    """BASELINE config 3 (decode) or 4 (fused append + decode) through 32
    layers: fills the ring, times `steps` graph-replayed steps after `warmup`
    (time_steps) and returns the figures together with the live ring and the
    inputs (for the CPU baseline)."""
    from bmo_jetson_amd import KVRing

    H, D, W, L = 32, 128, 512, 32
    S = sessions or (64 if config == "cfg3" else 256)
    fused = config == "cfg4"
    from bmo_jetson_amd.synth import positions

    seed = 0xB0A00003 if config == "cfg3" else 0xB0A00004
    pos_host = np.array(positions(seed, S), dtype=np.int64)
    ring = KVRing(L, S, H, D, W)
    pos = torch.tensor(pos_host, dtype=torch.int32, device="cuda")
    q = torch.empty((L, S, H, D), device="cuda")
    out = torch.empty((L, S, H, D), device="cuda")
    if fused:
        kn = torch.empty((L, S, H, D), device="cuda")
        vn = torch.empty((L, S, H, D), device="cuda")

    def prepare():
        log(f"[bench] {config}: S={S} L={L} H={H} D={D} W={W} fused={fused}; filling ring")
        t_fill = time.time()
        # cfg4 appends the token at pos, so the ring holds the window before it
        fill_ring(torch, ring, L, S, H, D, W, pos_host - (1 if fused else 0), seed)
        # q (layer, session, head, dim): stream seed + 2; cfg4's new K/V rows:
        # streams seed + 3, seed + 4
        from bmo_jetson_amd.synth import fill_normal
        st = torch.cuda.current_stream()
        fill_normal(q, seed + 2, stream=st)
        if fused:
            fill_normal(kn, seed + 3, stream=st)
            fill_normal(vn, seed + 4, stream=st)
        torch.cuda.synchronize()
        log(f"[bench] ring {ring.nbytes / 1e9:.2f} GB filled in {time.time() - t_fill:.1f} s")

    def launch_layer(layer, st):
        if fused:
            ring.append_decode(layer, pos, q[layer], kn[layer], vn[layer], out[layer], H, stream=st)
        else:
            ring.decode(layer, pos, q[layer], out[layer], H, stream=st)

    ms_per_step, per_step = time_steps(torch, launch_layer, L, steps, warmup, prepare)
    launch_ms = ms_per_step / L
    per_step_bytes = unit_bytes(H, D, W) * S * L
    if fused:
        per_step_bytes += fused_extra_bytes(H, D) * S * L
    value = per_step_bytes / (ms_per_step * 1e-3) / 1e9
    launch_bytes = per_step_bytes // L
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    log(f"[bench] {config}: {ms_per_step:.3f} ms/step, {value:.1f} GB/s; per launch "
        f"{launch_ms * 1e3:.2f} us -> {achieved:.1f} GB/s")
    return {
        "H": H, "D": D, "W": W, "L": L, "S": S,
        "ring": ring, "pos_host": pos_host, "q": q, "out": out,
        "value": round(value, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms_per_step, 4),
        "step_ms_dist": {"median": round(float(np.median(per_step)), 4),
                         "min": round(min(per_step), 4), "max": round(max(per_step), 4),
                         "n": len(per_step), "note": "separate replays after the timed region"},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "config": {
            "workload": (f"{config}: Q4_0 ring {'fused append+' if fused else ''}decode "
                         f"attention, S={S} sessions x L={L} layers, H={H} x D={D}, W={W}, "
                         f"pos~U[512,4096), 1% x8 outliers"),
            "sessions": S, "layers": L, "heads": H, "head_dim": D, "window": W,
            "bytes_per_step": per_step_bytes, "launches_per_step": L,
            "parallelism": "none (1 GPU; sessions would shard across GPUs)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(config),
            "kernel": "decode_kernel<128, 1, 2, %s>" % ("true" if fused else "false"),
            "launch_us": round(launch_ms * 1e3, 3),
            "bytes_per_launch": launch_bytes,
        },
    }


def cpu_baseline(torch, ring, L, S, H, D, W, pos_host, q_dev, out_dev, budget_s):
    """Times two CPU restatements on host threads over a sample of the same
    ring (layer 0, the first n sessions), each for about budget_s / 2:
      - value: the arithmetic of ggml's CPU flash attention over Q4_0 K/V,
        the backend the reference's lazy path reaches through
        ggml_flash_attn_ext (src/bmo_compute.cpp:2410-2412): q to Q8_0, AVX2
        Q4_0 x Q8_0 dot products, online softmax, V dequantized to fp32
        (oracle/cpu_ggml_style.c);
      - eager_loop_*: the reference's own scalar CPU decode loop
        (src/bmo_compute.cpp:927-970) restated in fp32 (oracle/cpu_baseline.c).
    Both outputs are compared with the GPU output of those sessions."""
    import oracle

    # The GPU box grants one GPU's job a share of 16 host CPUs, whatever the
    # affinity mask or nproc show; the pool is sized to that share.
    host_cpus = len(os.sched_getaffinity(0))
    n_threads = max(1, min(16, host_cpus))

    def stripes(n):
        kc = np.zeros((n, H, W, D // 32), dtype=oracle.BLOCK_DTYPE)
        vc = np.zeros_like(kc)
        for s in range(n):
            for which, dst in ((0, kc), (1, vc)):
                raw = ring.export_q4_0(0, s, which, 0, W)  # [W][H][nblk][18]
                dst[s] = np.ascontiguousarray(raw.transpose(1, 0, 2, 3)).view(oracle.BLOCK_DTYPE)[..., 0]
        return kc, vc

    q_host = q_dev[0].float().cpu().numpy()  # layer 0: [S][H][D]
    gpu_all = out_dev[0].float().cpu().numpy()
    kc1, vc1 = stripes(1)

    def timed(run, budget):
        secs1, _ = run(kc1, vc1, pos_host[:1], q_host[:1], H, 1, 1)
        # size the multi-thread sample to ~budget
        per_unit_mt = max(secs1 / max(1, n_threads * 0.8), 1e-4)
        n_sess = int(min(S, max(n_threads, round(budget / per_unit_mt))))
        iters = max(1, int(budget / (per_unit_mt * n_sess)))
        kc, vc = stripes(n_sess)
        secs, out = run(kc, vc, pos_host[:n_sess], q_host[:n_sess], H, n_threads, iters)
        secs_1t, _ = run(kc[:1], vc[:1], pos_host[:1], q_host[:1], H, 1, 3)
        err = np.abs(gpu_all[:n_sess] - out)
        return {"GBps": round(unit_bytes(H, D, W) * n_sess * iters / secs / 1e9, 3),
                "sample": f"layer 0 of the cfg3 ring, {n_sess} sessions x {H} heads x W={W}, "
                          f"{iters} pass(es), {n_threads} threads, {secs:.1f} s",
                "single_thread_GBps": round(unit_bytes(H, D, W) * 3 / secs_1t / 1e9, 3),
                "single_thread_us_per_layer_b1": round(secs_1t / 3 * 1e6, 1),
                "max_abs_vs_gpu": float(err.max())}

    gg = timed(oracle.cpu_ggml_style_run, budget_s / 2)
    eager = timed(oracle.cpu_baseline_run, budget_s / 2)
    return {
        "value": gg["GBps"],
        "unit": "GB/s",
        "cores": n_threads,
        "host_cpus_visible": host_cpus,
        "nproc": os.cpu_count(),
        "cores_note": "threads used = the 16-CPU share the GPU box grants one GPU's job",
        "kind": "port",
        "sample": gg["sample"],
        "single_thread_GBps": gg["single_thread_GBps"],
        "single_thread_us_per_layer_b1": gg["single_thread_us_per_layer_b1"],
        "max_abs_vs_gpu": gg["max_abs_vs_gpu"],
        "what": "restatement of ggml's CPU flash attention over Q4_0 K/V (q to Q8_0, AVX2 "
                "Q4_0 x Q8_0 dots, online softmax, fp32 V), the backend of "
                "src/bmo_compute.cpp:2410-2412; ggml itself is not available offline",
        "eager_loop_port": dict(eager, what="fp32 restatement of the reference's scalar CPU "
                                            "decode loop (src/bmo_compute.cpp:927-970)"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=300,
                    help="untimed graph replays right before the timed region (300 cfg3 steps: about 0.25 s)")
    ap.add_argument("--config", default="cfg3", choices=["cfg3", "cfg4"])
    ap.add_argument("--sessions", type=int, default=None, help="override S (testing)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b1", action="store_true")
    ap.add_argument("--no-cfg4", action="store_true",
                    help="skip the BASELINE config 4 leg (fused append + decode, 256 sessions)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run the cfg5 chunked-prefill leg and print its JSON (profiling)")
    ap.add_argument("--latency-only", action="store_true",
                    help="only run the B=1 and depformer legs (rocprof of the latency kernels)")
    ap.add_argument("--prefill-phases", action="store_true",
                    help="only run the cfg5 prefill phase timings of the diagnostic library "
                         "libbmo_attn_phases.so and print their JSON")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only run the Q4_0 GEMV leg and print its JSON (profiling)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run a plain device copy of this size (rocprof PMC calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this path runs on one GPU: sessions shard across GPUs with no "
                          "exchange, so the figure is the one-GPU number; --gpus N>1 is not "
                          "supported"}))
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib * (1 << 20) // 4
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4}))
        return

    if args.prefill_phases:
        from bmo_jetson_amd import _lib
        _lib.LIB_PATH = os.path.join(_lib.PKG_DIR, "libbmo_attn_phases.so")
        print(json.dumps({"prefill_phases": prefill_phases(torch)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": bench_prefill(torch)}), flush=True)
        return
    if args.gemv_only:
        print(json.dumps({"gemv": bench_gemv(torch)}), flush=True)
        return
    if args.latency_only:
        print(json.dumps({"b1": bench_b1(torch), "depformer": bench_depformer(torch)}), flush=True)
        return

    run = run_decode(torch, args.config, args.steps, args.warmup, args.sessions)
    H, D, W, L, S = run["H"], run["D"], run["W"], run["L"], run["S"]
    result = {
        "metric": METRIC,
        "value": run["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": run["ms_per_step"],
        "step_ms_dist": run["step_ms_dist"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": run["config"],
        "hbm_frac": run["hbm_frac"],
        "roofline": run["roofline"],
    }
    # the read probe over each layer's ring stripes (the window bytes the
    # decode launch of that layer reads; q and out, 1 MB each at cfg3, are
    # not in it): the ceiling of one launch
    ring0 = run["ring"]
    slice_bytes = ring0.nbytes // L
    result["read_ceiling"] = read_ceiling(torch, [ring0.k_base + i * slice_bytes for i in range(L)],
                                          slice_bytes)
    result["read_ceiling"]["note"] = ("libbmo_synth.so read probe over one layer's ring stripes per launch, "
                                      "32 launches per graph; compare the decode's launch_us")
    log(f"[bench] read ceiling: {result['read_ceiling']}")
    if args.config == "cfg3" and not args.no_cfg4:
        # BASELINE config 4 (fused append + decode, 256 sessions) at the same
        # step count; its 19.3 GB ring is freed before the other legs
        c4 = run_decode(torch, "cfg4", args.steps, args.warmup, None)
        c4["ring"].close()
        result["cfg4"] = {k: c4[k] for k in ("value", "unit", "ms_per_step", "step_ms_dist",
                                             "hbm_frac", "roofline", "config")}
        del c4
        torch.cuda.empty_cache()
    ring, pos_host, q, out = run["ring"], run["pos_host"], run["q"], run["out"]

    if not args.no_b1:
        result["b1"] = bench_b1(torch)
        log(f"[bench] B=1: {result['b1']}")
        result["depformer"] = bench_depformer(torch)
        log(f"[bench] depformer: {result['depformer']}")
        result["prefill"] = bench_prefill(torch)
        log(f"[bench] prefill: {result['prefill']}")
        result["gemv"] = bench_gemv(torch)
        log(f"[bench] gemv: {result['gemv']}")
    if not args.no_cpu:
        log("[bench] timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(torch, ring, L, S, H, D, W, pos_host, q, out,
                                              args.cpu_seconds)
    ring.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
