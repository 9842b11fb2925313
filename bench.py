"""Benchmark of the GDN-2 hip backend on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode] [--no-layer]

Headline (BASELINE.json ``metric``): prefill tokens/s at BASELINE config 1
(B=2 S=4096 H=16 DK=DV=128, bf16 q,k,v,b,w, fp32 g, synthetic data with the
config's distributions). A step is one prefill of the batch through the C ABI:
``gdn2_hip_chunk_local`` then ``gdn2_hip_prefill_scan`` with inputs already
resident in HBM. Two input sets are alternated so the 256 MB Infinity Cache
cannot hold a step's working set.

Also reported: decode state GB/s for BASELINE configs 2 (decode_step, B=64,
64 calls) and 3 (decode_multi n=8, B=32), rotating enough independent states
(> 256 MB in total) that every call streams its state from HBM, and the CPU
baseline: the oracle's chunkwise torch path on the host cores, and the
GatedDeltaNet2 layer at BASELINE config 4 (segmented prefill + 128 steps).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch
import torch.nn.functional as F

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, GB/s
BF16_DENSE_TFLOPS = 2500.0       # MI355X dense bf16 MFMA

# BASELINE config 1
B1, S1, H1, D1 = 2, 4096, 16, 128
# algorithmic bytes of one config-1 prefill: q,k,v,b,w bf16 + g fp32 in, o bf16 out,
# final fp32 state out (no initial state)
ALG_BYTES_PREFILL = (5 * B1 * S1 * H1 * D1 * 2) + (B1 * S1 * H1 * D1 * 4) \
    + (B1 * S1 * H1 * D1 * 2) + (B1 * H1 * D1 * D1 * 4)
# dense GEMM flops of the chunkwise form per 64-token chunk (QK^T, EK^T, Ai E,
# Ai Z, W S, Qg S, Aqk Un, KG^T Un)
BS = 64
FLOPS_PER_CHUNK = 2 * BS * BS * (3 * D1 + 2 * D1) + 6 * BS * D1 * D1
ALG_FLOPS_PREFILL = FLOPS_PER_CHUNK * B1 * H1 * (S1 // BS)
# the reference benchmark's count (bench/bench_gdn2.py:55-64): four [BS, BS] x
# [BS, D] products and two [BS, DK] x [DK, DV] products per chunk
REF_FLOPS_PREFILL = (2 * BS * BS * (2 * D1 + 2 * D1) + 2 * 2 * BS * D1 * D1) * B1 * H1 * (S1 // BS)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cfg_inputs(B, S, H, DK, DV, seed, device="cuda", dtype=torch.bfloat16):
    """q,k ~ N(0,1) L2-normalised, v ~ N(0,1), g = logsigmoid(N(0,1)), b,w = sigmoid(N(0,1))."""
    gen = torch.Generator(device=device).manual_seed(seed)
    kw = dict(generator=gen, device=device, dtype=torch.float32)
    q = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1).to(dtype)
    v = torch.randn(B, S, H, DV, **kw).to(dtype)
    g = F.logsigmoid(torch.randn(B, S, H, DK, **kw))
    b = torch.sigmoid(torch.randn(B, S, H, DK, **kw)).to(dtype)
    w = torch.sigmoid(torch.randn(B, S, H, DV, **kw)).to(dtype)
    return q, k, v, g, b, w


def bench_prefill(steps, warmup):
    from gdt2_tilelang_amd import _hip

    lib = _hip.lib()
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream()
    sp = _hip.stream_of(dev)
    sets = [cfg_inputs(B1, S1, H1, D1, D1, seed=s) for s in (11, 12)]
    n_tok = S1
    ws_bytes = lib.gdn2_hip_prefill_workspace_bytes(B1, H1, D1, n_tok)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    o = torch.empty(B1, S1, H1, D1, dtype=torch.bfloat16, device=dev)
    st = torch.empty(B1, H1, D1, D1, dtype=torch.float32, device=dev)
    P = _hip.ptr
    scale = D1 ** -0.5

    def step(i, ev=None):
        q, k, v, g, b, w = sets[i % 2]
        if ev is not None:
            ev[0].record(stream)
        _hip.check(lib.gdn2_hip_chunk_local(P(q), P(k), P(b), P(g), 1, P(ws), B1, H1, D1, S1, 0, n_tok,
                                            scale, sp), "chunk_local")
        if ev is not None:
            ev[1].record(stream)
        _hip.check(lib.gdn2_hip_prefill_scan(P(v), P(w), 1, P(ws), None, P(st), P(o), 1, B1, H1, H1, D1, D1,
                                             S1, 0, n_tok, sp), "prefill_scan")
        if ev is not None:
            ev[2].record(stream)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    # whole-step timing (no per-kernel events inside)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    # per-kernel timing with events around each launch on the launch stream
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    cl = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    sc = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
    return ms_step, cl, sc


def bench_public_prefill(reps=20):
    """Config 1 through the public ``gdn2_prefill`` (Python checks, the
    workspace and outputs from torch's caching allocator, both kernels), as a
    caller of the package sees it; the headline times the C ABI pair on
    preallocated buffers."""
    from gdt2_tilelang_amd import gdn2_prefill

    sets = [cfg_inputs(B1, S1, H1, D1, D1, seed=s) for s in (11, 12)]
    for i in range(3):
        gdn2_prefill(*sets[i % 2])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(reps):
        gdn2_prefill(*sets[i % 2])
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps * 1e3
    ms = e0.elapsed_time(e1) / reps
    return {"entry": "gdn2_prefill(q, k, v, g, b, w) at config 1, bf16 o, fp32 state",
            "ms_per_call": round(ms, 5), "host_wall_ms_per_call": round(wall, 5),
            "tokens_per_s": round(B1 * S1 / (ms * 1e-3), 1)}


def bench_varlen(reps=20, nseq=16):
    """Config 1's 8192 tokens packed as nseq sequences of seeded random lengths
    (one gdn2_hip_prefill_varlen call: one chunk-local and one scan launch),
    against the same sequences as separate prefill calls."""
    from gdt2_tilelang_amd import _hip

    lib = _hip.lib()
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream()
    sp = _hip.stream_of(dev)
    T = B1 * S1
    gen = torch.Generator().manual_seed(21)
    cuts = sorted((torch.randperm(T - 1, generator=gen)[:nseq - 1] + 1).tolist())
    cu = [0] + cuts + [T]
    lens = [cu[i + 1] - cu[i] for i in range(nseq)]
    q, k, v, g, b, w = cfg_inputs(1, T, H1, D1, D1, seed=13)
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.gdn2_hip_prefill_varlen_workspace_bytes(nseq, H1, D1, T), dtype=torch.uint8, device=dev)
    ws1 = torch.empty(lib.gdn2_hip_prefill_workspace_bytes(1, H1, D1, max(lens)), dtype=torch.uint8, device=dev)
    o = torch.empty(1, T, H1, D1, dtype=torch.bfloat16, device=dev)
    st = torch.empty(nseq, H1, D1, D1, dtype=torch.float32, device=dev)
    P = _hip.ptr
    scale = D1 ** -0.5

    def packed():
        _hip.check(lib.gdn2_hip_prefill_varlen(P(q), P(k), P(v), P(g), P(b), P(w), 1, P(cu_dev), nseq, None,
                                               P(st), P(o), 1, P(ws), H1, H1, D1, D1, T, scale, sp), "varlen")

    def separate():
        for i in range(nseq):
            _hip.check(lib.gdn2_hip_prefill_chunks(
                P(q), P(k), P(v), P(g), P(b), P(w), 1, None, P(st[i]), P(o), 1, P(ws1), 1, H1, H1, D1, D1,
                T, cu[i], lens[i], scale, sp), "prefill_chunks")

    res = {}
    for name, fn in (("packed", packed), ("separate_calls", separate)):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / reps * 1e3
    return {"sequences": nseq, "tokens": T, "min_len": min(lens), "max_len": max(lens),
            "heads": H1, "head_dim": D1,
            "packed_us": round(res["packed"], 1), "packed_tokens_per_s": round(T / (res["packed"] * 1e-6), 1),
            "separate_calls_us": round(res["separate_calls"], 1)}


def bench_backward(reps=5):
    """Training backward at config 1's shape (bf16 inputs, fp32 arithmetic):
    chunk_gdn2_bwd with no initial state and no final-state gradient, the
    common training case; timed with HIP events on the current stream."""
    from gdt2_tilelang_amd import chunk_gdn2_bwd

    q, k, v, g, b, w = cfg_inputs(B1, S1, H1, D1, D1, seed=17)
    do = torch.randn(B1, S1, H1, D1, device="cuda", generator=torch.Generator("cuda").manual_seed(18)).bfloat16()
    for _ in range(2):
        chunk_gdn2_bwd(q, k, v, g, b, w, None, None, do, None)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        chunk_gdn2_bwd(q, k, v, g, b, w, None, None, do, None)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"workload": "chunk_gdn2_bwd, BASELINE config 1 shape (B=2 S=4096 H=16 DK=DV=128, bf16 in, fp32 "
                        "arithmetic, dq dk dv dg db dw)", "ms": round(ms, 3),
            "tokens_per_s": round(B1 * S1 / (ms * 1e-3), 1), "reps": reps}


def bench_decode(B, n, calls, steps_per_buf_min, H=16, D=128):
    """Average µs per decode call with rotating states (> MALL) for config 2/3.

    The headline figure replays the `calls` launches from one HIP graph, so it
    is the GPU time per call: a serving loop launches decode that way, and a
    Python loop of ctypes launches can take longer per call than the kernel.
    The eager (Python loop) figure is reported beside it."""
    from gdt2_tilelang_amd import _hip

    lib = _hip.lib()
    dev = torch.device("cuda")
    state_bytes = B * H * D * D * 4
    nbuf = max(2, -(-320 * 2 ** 20 // state_bytes))      # > 256 MB Infinity Cache in total
    states = [torch.randn(B, H, D, D, device=dev) * 0.1 for _ in range(nbuf)]
    tok = [cfg_inputs(B, n, H, D, D, seed=100 + i) for i in range(4)]
    o = torch.empty(B, n, H, D, dtype=torch.bfloat16, device=dev)
    P = _hip.ptr
    scale = D ** -0.5

    def call(i):
        q, k, v, g, b, w = tok[i % 4]
        _hip.check(lib.gdn2_hip_decode(P(q), P(k), P(v), P(g), P(b), P(w), 1, P(states[i % nbuf]), P(o), 1,
                                       B, H, H, D, D, n, 0, n, scale, _hip.stream_of(dev)), "decode")

    for i in range(2 * nbuf):
        call(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(calls):
        call(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us_eager = e0.elapsed_time(e1) * 1e3 / calls

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(calls):
            call(i)
    graph.replay()
    torch.cuda.synchronize()
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    reps = 5
    g0.record()
    for _ in range(reps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    us = g0.elapsed_time(g1) * 1e3 / (reps * calls)
    st_traffic = 2 * state_bytes
    tok_bytes = B * n * H * D * (4 * 2 + 4 + 2 * 2) + B * n * H * D * 2   # q,k,b bf16 + g fp32 + v,w + o
    gbs = st_traffic / (us * 1e-6) / 1e9
    return dict(B=B, n=n, H=H, DK=D, DV=D, calls=calls, state_buffers=nbuf, us_per_call=round(us, 3),
                us_per_call_eager=round(us_eager, 3), timing="HIP graph replay of the calls",
                state_GBps=round(gbs, 1), state_frac_of_peak=round(gbs / HBM_PEAK_GBS, 4),
                total_GBps=round((st_traffic + tok_bytes) / (us * 1e-6) / 1e9, 1),
                tokens_per_s=round(B * n / (us * 1e-6), 1))


def bench_layer(reps=3):
    """a GatedDeltaNet2 layer (hidden 2048, 16 value / 8 key
    heads, head dims 128, random-init bf16 weights, x ~ N(0,1), B=1) prefills a
    ragged 32700-token prompt in 4 segments, passing the cache back between
    them, then decodes 128 steps through ``GatedDeltaNet2.step``. Eager calls,
    as a user of the layer makes them; best of ``reps`` runs."""
    from gdt2_tilelang_amd import GatedDeltaNet2, GatedDeltaNet2Config

    torch.manual_seed(0)
    cfg = GatedDeltaNet2Config(hidden_size=2048, num_heads=16, num_kv_heads=8, head_dim_k=128,
                               head_dim_v=128)
    layer = GatedDeltaNet2(cfg).cuda().to(torch.bfloat16).eval()
    S, steps = 32700, 128
    gen = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(1, S + steps, 2048, device="cuda", generator=gen).to(torch.bfloat16)
    bounds = [0, 8175, 16350, 24525, S]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def run():
        cache = None
        ev[0].record()
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            _, cache = layer.prefill(x[:, lo:hi], cache)
        ev[1].record()
        for t in range(steps):
            layer.step(x[:, S + t], cache)
        ev[2].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])

    run()
    pf, dc = min(run() for _ in range(reps))

    # the same 128 step() calls captured once in a HIP graph and replayed: the
    # GPU time of a step without the per-call host work (Python, ctypes, launches)
    cache = None
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        _, cache = layer.prefill(x[:, lo:hi], cache)
    xs = x[:, S:S + steps].clone()
    for t in range(3):                                  # warm the allocator and caches outside the capture
        layer.step(xs[:, t], cache)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for t in range(steps):
            layer.step(xs[:, t], cache)
    graph.replay()
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(reps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    dg = g0.elapsed_time(g1) / reps
    return dict(workload="GatedDeltaNet2 layer, BASELINE config 4: hidden 2048, H=16 HK=8 DK=DV=128, "
                         "bf16, B=1, 32700-token prompt in 4 segments then 128 step() calls",
                prefill_ms=round(pf, 3), prefill_tokens_per_s=round(S / (pf * 1e-3), 1),
                decode_ms_128_steps=round(dc, 3), decode_steps_per_s=round(steps / (dc * 1e-3), 1),
                decode_graph_ms_128_steps=round(dg, 3), decode_graph_steps_per_s=round(steps / (dg * 1e-3), 1),
                decode_graph_timing="the 128 step() calls captured in one HIP graph, replayed %d times" % reps,
                timing="eager Python calls, HIP events, best of %d" % reps)


def measure_copy_peak(reps=10, nbytes=2 ** 30):
    """Measured streaming-copy rate of this GPU: a plain device copy of
    ``nbytes`` (torch ``copy_``, read + write), timed with HIP events; the
    practical HBM ceiling each roofline fraction is also reported against."""
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return {"GBps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "bytes_read_plus_written": 2 * nbytes,
            "us_per_copy": round(ms * 1e3, 1),
            "how": "torch dst.copy_(src) of 1 GiB fp32, %d copies timed with HIP events" % reps}


def decode_sweep(B, ns=(1, 2, 4, 8, 16), copy_gbps=None):
    """State GB/s over tokens per call, the reference's decode benchmark sweep
    (bench/bench_decode.py:57, state bytes as its :71), with rotated states."""
    rows = []
    for n in ns:
        r = bench_decode(B, n, calls=64, steps_per_buf_min=1)
        row = {"n": n, "us_per_call": r["us_per_call"], "us_per_token": round(r["us_per_call"] / n, 3),
               "state_GBps": r["state_GBps"], "state_frac_of_peak": r["state_frac_of_peak"]}
        if copy_gbps:
            row["state_frac_of_measured_copy"] = round(r["state_GBps"] / copy_gbps, 4)
        rows.append(row)
    return {"B": B, "H": 16, "DK": 128, "DV": 128, "dtype": "bf16 tokens, fp32 state", "rows": rows}


def cpu_model():
    """The host CPU's model string (``/proc/cpuinfo``), or the platform's."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "host CPU"


def _timed(fn, budget_s, max_reps):
    """(reps, seconds): run fn until budget_s is spent or max_reps reached."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= max_reps:
            return reps, el


def cpu_baseline(budget_s=8.0):
    """The oracle's restatements of the reference's torch paths on the host
    cores, one bounded sample per BASELINE config (kind "port": the
    reference's Python does not travel to the GPU box):

    * config 1: the chunkwise torch form (reference gdn2/reference.py:168-261)
      on full config-1 prefills -- the headline comparison;
    * configs 2 and 3: the per-token torch decode loop
      (reference gdn2/inference.py:337-345) on the full-size batch;
    * config 4: the torch layer (reference gdn2/attention.py:360-479) on a
      2048-token prompt segment and 16 single-token decode calls.
    """
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle
    from oracle import chunk_gdn2

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cpu = cpu_model()

    def f32(ins):
        q, k, v, g, b, w = ins
        return tuple(t.float() for t in (q, k, v)) + (g,) + tuple(t.float() for t in (b, w))

    ins = f32(cfg_inputs(B1, S1, H1, D1, D1, seed=11, device="cpu"))
    chunk_gdn2(*(t[:, :256] for t in ins))          # warm-up
    reps, el = _timed(lambda: chunk_gdn2(*ins, output_final_state=True), budget_s, 20)
    out = {"value": round(reps * B1 * S1 / el, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
           "cpu_model": cpu,
           "sample": f"{reps} full config-1 prefills (B=2 S=4096 H=16 D=128, fp32 torch chunkwise "
                     f"oracle) in {el:.1f} s on {threads} threads of {cpu}"}
    per = {}
    for name, B, n in (("config2_decode_step", 64, 1), ("config3_decode_multi_n8", 32, 8)):
        tok = f32(cfg_inputs(B, n, H1, D1, D1, seed=100, device="cpu"))
        st = torch.randn(B, H1, D1, D1, generator=torch.Generator().manual_seed(5)) * 0.1
        oracle.decode_loop(*tok, st, None)
        reps, el = _timed(lambda: oracle.decode_loop(*tok, st, None), budget_s / 3, 400)
        us = el / reps * 1e6
        gbs = 2 * B * H1 * D1 * D1 * 4 / (us * 1e-6) / 1e9
        per[name] = {"us_per_call": round(us, 1), "state_GBps": round(gbs, 2),
                     "tokens_per_s": round(B * n / (us * 1e-6), 1),
                     "sample": f"{reps} calls of the fp32 torch per-token decode loop, B={B} n={n} H=16 D=128"}
    from gdt2_tilelang_amd import GatedDeltaNet2, GatedDeltaNet2Config
    torch.manual_seed(0)
    cfg = GatedDeltaNet2Config(hidden_size=2048, num_heads=16, num_kv_heads=8, head_dim_k=128, head_dim_v=128)
    ref = oracle.LayerOracle(GatedDeltaNet2(cfg).state_dict(), 2048, 16, 8, 128, 128)
    x = torch.randn(1, 2048 + 16, 2048, generator=torch.Generator().manual_seed(1))
    t0 = time.perf_counter()
    _, cache = ref.prefill(x[:, :2048])
    t_pf = time.perf_counter() - t0
    t0 = time.perf_counter()
    for i in range(16):
        ref.decode(x[:, 2048 + i:2049 + i], cache)
    t_dc = time.perf_counter() - t0
    per["config4_layer"] = {"prefill_tokens_per_s": round(2048 / t_pf, 1), "decode_steps_per_s": round(16 / t_dc, 1),
                            "sample": "fp32 torch layer (hidden 2048, H=16 HK=8, D=128, B=1): one 2048-token "
                                      f"prompt segment in {t_pf:.2f} s, 16 one-token decode calls in {t_dc:.2f} s"}
    out["configs"] = per
    return out


def read_traffic():
    """HBM bytes per prefill step from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "hbm_traffic_pmc.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_step:"):
                return float(line.split(":")[1])
    return None


def read_mfma_busy():
    """MFMA busy fraction per prefill kernel from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mfma_busy_pmc.txt")
    if not os.path.exists(path):
        return None
    out = {}
    with open(path) as f:
        for line in f:
            if "(prefill, config 1)" in line and "%" in line:
                name = "chunk_local" if "chunk_local" in line else "scan"
                pct = [t for t in line.split() if t.endswith("%")][0]
                out[name] = round(float(pct[:-1]) / 100, 4)
    return out or None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode configs")
    ap.add_argument("--prefill-only", action="store_true", help="prefill steps only (for profilers)")
    ap.add_argument("--decode-only", action="store_true", help="decode configs only (for profilers)")
    ap.add_argument("--no-layer", action="store_true", help="skip the config-4 layer run")
    ap.add_argument("--no-varlen", action="store_true", help="skip the packed-sequence prefill run")
    ap.add_argument("--varlen-only", action="store_true", help="packed-sequence prefill run only (for profilers)")
    ap.add_argument("--layer-only", action="store_true", help="config-4 layer run only (for profilers)")
    ap.add_argument("--no-backward", action="store_true", help="skip the training-backward run")
    ap.add_argument("--backward-only", action="store_true", help="training backward only (for profilers)")
    ap.add_argument("--decode-sweep-only", action="store_true", help="copy peak + decode n-sweep only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="three plain 1 GiB device copies (scales rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the GDN-2 path shards by "
                                   "batch/head with no exchange between GPUs, so one GPU's share is the same kernels at a smaller shape; --gpus must be 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(2)

    log(f"device: {torch.cuda.get_device_name()}")
    if args.decode_sweep_only:
        copy = measure_copy_peak()
        log(json.dumps({"hbm_copy": copy, "sweep_B8": decode_sweep(8, copy_gbps=copy["GBps"]),
                        "sweep_B32": decode_sweep(32, copy_gbps=copy["GBps"])}))
        return
    if args.copy_calibration:
        src = torch.ones(2 ** 28, device="cuda")          # 1 GiB fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 1073741824 bytes read + written")
        return
    if args.decode_only:
        log(json.dumps({"config2_decode_step": bench_decode(64, 1, calls=64, steps_per_buf_min=1),
                        "config3_decode_multi_n8": bench_decode(32, 8, calls=64, steps_per_buf_min=1)}))
        return
    if args.layer_only:
        log(json.dumps(bench_layer()))
        return
    if args.varlen_only:
        log(json.dumps(bench_varlen()))
        return
    if args.backward_only:
        log(json.dumps(bench_backward()))
        return
    ms_step, cl_ms, sc_ms = bench_prefill(args.steps, args.warmup)
    if args.prefill_only:
        log(f"prefill {ms_step * 1e3:.1f} us/step (chunk_local {cl_ms * 1e3:.1f}, scan {sc_ms * 1e3:.1f})")
        return
    copy = measure_copy_peak()
    copy_gbps = copy["GBps"]
    tokens = B1 * S1
    value = tokens / (ms_step * 1e-3)
    kern_s = (cl_ms + sc_ms) * 1e-3
    achieved = ALG_BYTES_PREFILL / kern_s / 1e9
    traffic = read_traffic()
    out = {
        "metric": "prefill tokens/s (S=4096) + decode state GB/s vs HBM peak, 1 MI355X",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "gdn2 prefill, BASELINE config 1: B=2 S=4096 H=16 DK=DV=128, "
                               "bf16 q,k,v,b,w + fp32 g in, bf16 o + fp32 state out, chunk 64",
                   "global_batch": B1, "seq_len": S1, "heads": H1, "head_dim": D1,
                   "arithmetic": "bf16 and fp16 MFMA (hi/lo splits where precision needs it), fp32 accumulate"},
        "roofline": {
            "bound": "hbm",
            "kernel": "prefill step = gdn2 chunk_local_m_kernel + scan_e_kernel (DK=128 factored transition records)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "frac_of_measured_copy": round(achieved / copy_gbps, 4),
            "hbm_copy_GBps": copy_gbps,
            "traffic": traffic,
            "traffic_source": "profiles/hbm_traffic_pmc.txt (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of "
                              "this bench, committed; not counted in this run)",
            "algorithmic_bytes": ALG_BYTES_PREFILL,
            "kernel_us": {"chunk_local": round(cl_ms * 1e3, 2), "scan": round(sc_ms * 1e3, 2)},
            "gemm_tflops": round(ALG_FLOPS_PREFILL / kern_s / 1e12, 1),
            "gemm_frac_of_bf16_peak": round(ALG_FLOPS_PREFILL / kern_s / 1e12 / BF16_DENSE_TFLOPS, 4),
            "gemm_gflop_per_step": round(ALG_FLOPS_PREFILL / 1e9, 2),
            "reference_formula_gflop_per_step": round(REF_FLOPS_PREFILL / 1e9, 2),
            "reference_formula_tflops": round(REF_FLOPS_PREFILL / kern_s / 1e12, 1),
            "mfma_busy_pmc": read_mfma_busy(),
            "mfma_busy_source": "profiles/mfma_busy_pmc.txt (rocprofv3 --pmc run of this bench, committed; "
                                "not counted in this run)",
        },
        "hbm_copy": copy,
    }
    if not args.no_decode:
        out["decode"] = {
            "config2_decode_step": bench_decode(64, 1, calls=64, steps_per_buf_min=1),
            "config3_decode_multi_n8": bench_decode(32, 8, calls=64, steps_per_buf_min=1),
        }
        for r in out["decode"].values():
            r["state_frac_of_measured_copy"] = round(r["state_GBps"] / copy_gbps, 4)
        out["decode"]["sweep_reference_bench_B8"] = decode_sweep(8, copy_gbps=copy_gbps)
        out["decode"]["sweep_B32"] = decode_sweep(32, copy_gbps=copy_gbps)
    out["public_prefill"] = bench_public_prefill()
    if not args.no_varlen:
        out["varlen"] = bench_varlen()
    if not args.no_layer:
        out["layer"] = bench_layer()
    if not args.no_backward:
        out["backward"] = bench_backward()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
