#!/usr/bin/env python3
"""Benchmark of the Q4_K GEMM core on one MI355X.

Headline (BASELINE.json metric "Q4_K GEMV achieved HBM GB/s (% of peak) at M=1; MoE
decode-step us"): the north-star Q4_K GEMV, M=1, K=N=6144, fast mode.  One step = one GEMV
launch over one batch of synthetic input (weights + activation vector).  Inputs are resident
in HBM before timing; weights rotate over >= 1 GB of distinct copies so every launch streams
from HBM, not from the 256 MB Infinity Cache.  The K timed launches are captured in one HIP
graph and bracketed by HIP events on the launch stream.

Also reported (in "extra"): the MoE SwiGLU decode step (config 2) in us, the other BASELINE
configs, a streaming-read ceiling, a cache-hot (labelled) GEMV number, and launch-group
percentiles.  ``cpu_baseline`` times the repo's CPU restatement of the reference's path on
this host (bounded sample, extrapolated linearly in N).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu] [--no-extra]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV achieved HBM GB/s (% of peak) at M=1; MoE decode-step µs"
REPS = 7          # timed graph replays per measurement (the median is reported)
PEAK_GBS = 8000.0
Q4K = 12
BF16 = 30


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4k_bytes(N, K):
    return N * K // 256 * 144


def gen_q4k(n_rows, K, gen, device):
    """BASELINE config-0 distribution on the device: uniform bytes, d/dmin = fp16(|N(0,1)| 2^-8)."""
    import torch
    nb = n_rows * K // 256
    raw = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=device, generator=gen)
    hdr = (torch.randn((nb, 2), device=device, generator=gen).abs() * 2.0 ** -8).to(torch.float16)
    raw[:, 0:4] = hdr.view(torch.uint8).view(nb, 4)
    return raw.view(-1)


def time_graph(fn_list, reps=1, discard=1):
    """Capture fn_list into one graph, replay it `discard` times untimed and then `reps` times
    bracketed by HIP events on the replay stream; return ms per timed replay (list)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fn_list[:2]:
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fn_list:
            f()
    torch.cuda.synchronize()
    for _ in range(discard):
        g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1))
    return out, g


def pct(vals, q):
    import numpy as np
    return float(np.percentile(np.asarray(vals), q))


def time_eager(fn_list):
    """Eager launches bracketed by HIP events (lets a kernel tracer see every dispatch)."""
    import torch
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for f in fn_list:
        f()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def time_isolated(fn_list):
    """Each launch alone: HIP events on the launch stream around it, then a host sync before the
    next one, so no launch queues behind another (what a kernel tracer then sees per dispatch is
    the kernel's own duration).  Returns us per launch (list)."""
    import torch
    out = []
    for f in fn_list:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        f()
        e1.record()
        e1.synchronize()
        out.append(1000.0 * e0.elapsed_time(e1))
    return out


def bench_gemv(dev, torch, N, K, M, steps, warmup, rot_bytes, mode="fast", label="", eager=False, isolated=False):
    """Rotating-buffer GEMV timing.  Returns dict with us/launch, GB/s, percentiles, hot number.
    isolated: every launch alone (time_isolated), for kernel traces."""
    device = "cuda"
    wb = q4k_bytes(N, K)
    nbuf = max(2, math.ceil(rot_bytes / wb))
    gen = torch.Generator(device=device)
    gen.manual_seed(1234 + N + K + M)
    W = gen_q4k(nbuf * N, K, gen, device).view(nbuf, wb)
    X = (torch.randn((nbuf, M, K), device=device, generator=gen)).to(torch.bfloat16)
    Y = torch.empty((nbuf, M, N), dtype=torch.bfloat16, device=device)

    def launcher(i):
        j = i % nbuf
        return lambda: dev.gemv(Q4K, W[j], N, K, X[j], mode=mode, out=Y[j])

    for i in range(warmup):
        launcher(i)()
    torch.cuda.synchronize()
    if isolated:
        t = time_isolated([launcher(i) for i in range(steps)])
        alg = wb + 2 * K * M + 2 * N * M
        us = pct(t, 50)
        log(f"{label} isolated N={N} K={K} M={M} {mode}: median {us:.2f} us per launch alone (p10 {pct(t, 10):.2f}, "
            f"p90 {pct(t, 90):.2f}), {alg / (us * 1e-6) / 1e9:.0f} GB/s")
        return dict(N=N, K=K, M=M, mode=mode, us_per_launch=us, p10_us=pct(t, 10), p90_us=pct(t, 90),
                    gbs=alg / (us * 1e-6) / 1e9, alg_bytes=alg, weight_rotation_bytes=nbuf * wb,
                    timing="each launch alone: HIP events around it, host sync before the next")
    if eager:
        fns = [launcher(i) for i in range(steps)]
        total_ms = time_eager(fns)
        alg = wb + 2 * K * M + 2 * N * M
        us = 1000.0 * total_ms / steps
        log(f"{label} eager N={N} K={K} M={M} {mode}: {us:.2f} us/launch, {alg / (us * 1e-6) / 1e9:.0f} GB/s")
        return dict(N=N, K=K, M=M, mode=mode, us_per_launch=us, gbs=alg / (us * 1e-6) / 1e9, alg_bytes=alg,
                    weight_rotation_bytes=nbuf * wb, rotation_buffers=nbuf, pct_peak=100.0 * alg / (us * 1e-6) / 1e9 / PEAK_GBS,
                    timing="eager launches")
    # One graph of max(steps, nbuf) launches, so every rotation buffer is read once per replay
    # and the per-launch figure does not depend on --steps; one untimed replay, then the median
    # of REPS timed replays.
    nlaunch = max(steps, nbuf)
    ms, _ = time_graph([launcher(i) for i in range(nlaunch)], reps=REPS)
    per_launch_us = [1000.0 * t / nlaunch for t in ms]
    alg = wb + 2 * K * M + 2 * N * M
    us = pct(per_launch_us, 50)
    res = dict(N=N, K=K, M=M, mode=mode, us_per_launch=us, gbs=alg / (us * 1e-6) / 1e9,
               alg_bytes=alg, weight_rotation_bytes=nbuf * wb, rotation_buffers=nbuf, launches_per_replay=nlaunch,
               timed_replays=REPS, p10_us=pct(per_launch_us, 10), p50_us=us, p90_us=pct(per_launch_us, 90),
               min_us=min(per_launch_us))
    res["pct_peak"] = 100.0 * res["gbs"] / PEAK_GBS
    res["gemv_per_s"] = 1e6 / us
    res["tflops"] = 2.0 * M * N * K / (us * 1e-6) / 1e12
    hot = ""
    if mode != "ref":
        # cache-hot (labelled): the same buffer every launch
        hot_ms, _ = time_graph([(lambda: dev.gemv(Q4K, W[0], N, K, X[0], mode=mode, out=Y[0])) for _ in range(200)],
                               reps=3)
        res["hot_us"] = 1000.0 * pct(hot_ms, 50) / 200
        res["hot_gbs_cache_resident"] = alg / (res["hot_us"] * 1e-6) / 1e9
        hot = f"; hot {res['hot_us']:.2f} us"
    log(f"{label} N={N} K={K} M={M} {mode}: {us:.2f} us/launch, {res['gbs']:.0f} GB/s "
        f"({res['pct_peak']:.1f}% of 8 TB/s){hot}")
    del W, X, Y
    torch.cuda.empty_cache()
    return res


def bench_exact(dev, torch, rot_bytes):
    """The price of the reference's exact order (AIPU_MODE_REF: exact dequant, sequential fp32
    MAC in K order, bit-identical to tools/q4k_ref.py): the north-star GEMV and the verify
    batches of config 1, timed like the fast legs over one rotation of the weights."""
    out = {}
    for M in (1, 2, 4, 8):
        out[f"m{M}"] = bench_gemv(dev, torch, 6144, 6144, M, 1, 0, rot_bytes, mode="ref", label="exact order")
    return out


def bench_floor(dev, torch, N, K, rot_bytes, steps=1000):
    """What bounds the M = 1 GEMV at (N, K), each timed like the headline (one HIP graph of
    launches over rotating weights, median replay): an empty kernel with the GEMV kernel's
    launch shape, the kernel's weight-copy schedule alone (aipu_measure_gemv), and a plain
    streaming read of the same bytes per launch (aipu_stream_read)."""
    device = "cuda"
    wb = q4k_bytes(N, K)
    nbuf = max(2, math.ceil(rot_bytes / wb))
    gen = torch.Generator(device=device)
    gen.manual_seed(4321 + N + K)
    W = gen_q4k(nbuf * N, K, gen, device).view(nbuf, wb)
    X = (torch.randn((nbuf, 1, K), device=device, generator=gen)).to(torch.bfloat16)
    nlaunch = max(steps, nbuf)
    res = dict(N=N, K=K, alg_bytes=wb + 2 * K + 2 * N, launches_per_replay=nlaunch, timed_replays=REPS)
    for what in ("empty", "copy"):
        ms, _ = time_graph([(lambda j=i % nbuf: dev.measure_gemv(what, W[j], N, K, X[j])) for i in range(nlaunch)],
                           reps=REPS)
        res[f"{what}_us"] = 1000.0 * pct(ms, 50) / nlaunch
    res["copy_gbs"] = wb / (res["copy_us"] * 1e-6) / 1e9
    del W, X
    torch.cuda.empty_cache()
    rd = bench_stream_read_sized(dev, torch, res["alg_bytes"], rot_bytes)
    res["stream_read_us"] = rd["us_per_launch"]
    res["stream_read_gbs"] = rd["gbs"]
    log(f"floors N={N} K={K}: empty launch {res['empty_us']:.2f} us, copy schedule {res['copy_us']:.2f} us "
        f"({res['copy_gbs']:.0f} GB/s), stream read {res['stream_read_us']:.2f} us")
    return res


def bench_stream_read(dev, torch, nbytes=2 << 30, reps=10):
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    ms, _ = time_graph([lambda: dev.stream_read(buf, sink)], reps=reps)
    best = min(ms)
    del buf
    torch.cuda.empty_cache()
    return dict(bytes=nbytes, gbs_best=nbytes / (best * 1e-3) / 1e9, gbs_median=nbytes / (pct(ms, 50) * 1e-3) / 1e9)


def bench_stream_read_sized(dev, torch, nbytes, rot_bytes, steps=1000):
    """Read ceiling at one GEMV's size: `nbytes` per launch over rotating buffers."""
    nbuf = max(2, math.ceil(rot_bytes / nbytes))
    nb16 = (nbytes + 15) // 16 * 16
    buf = torch.ones(nbuf * nb16, dtype=torch.uint8, device="cuda").view(nbuf, nb16)
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    ms, _ = time_graph([(lambda j=i % nbuf: dev.stream_read(buf[j], sink)) for i in range(steps)], reps=2)
    us = 1000.0 * min(ms) / steps
    del buf
    torch.cuda.empty_cache()
    return dict(bytes=nb16, us_per_launch=us, gbs=nb16 / (us * 1e-6) / 1e9)


def bench_moe(dev, torch, steps, E=256, H=6144, I=2048, topk=8, mode="fast"):
    """bf16 router 6144->256, sigmoid top-8, Q4_K SwiGLU experts 6144<->2048."""
    device = "cuda"
    gen = torch.Generator(device=device)
    gen.manual_seed(99)
    ge = gen_q4k(E * I, H, gen, device)
    ue = gen_q4k(E * I, H, gen, device)
    de = gen_q4k(E * H, I, gen, device)
    rw = (torch.randn((E, H), device=device, generator=gen) * 0.05).to(torch.bfloat16)
    nx = 64
    X = (torch.randn((nx, H), device=device, generator=gen) * 0.05).to(torch.bfloat16)
    Y = torch.empty((nx, H), dtype=torch.bfloat16, device=device)
    ws = dev.moe_workspace(E, H, I, topk, device)
    sel = torch.empty(topk, dtype=torch.int32, device=device)
    sw = torch.empty(topk, dtype=torch.bfloat16, device=device)

    def step(i):
        j = i % nx
        return lambda: dev.moe_swiglu_decode(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, X[j], mode=mode,
                                             workspace=ws, out=Y[j], sel_out=(sel, sw))

    for i in range(3):
        step(i)()
    torch.cuda.synchronize()
    ms, _ = time_graph([step(i) for i in range(steps)], reps=REPS)
    us = [1000.0 * t / steps for t in ms]
    per_expert = 3 * q4k_bytes(I, H)
    alg = E * H * 2 + topk * per_expert + 2 * H * 2
    med = pct(us, 50)
    res = dict(E=E, H=H, I=I, topk=topk, mode=mode, us_per_step=med, us_min=min(us), us_p90=pct(us, 90),
               alg_bytes=alg, gbs=alg / (med * 1e-6) / 1e9, expert_bytes_stored=3 * E * q4k_bytes(I, H),
               timing=f"median of {REPS} replays of one HIP graph of {steps} steps (router -> top-8 -> "
                      f"gate/up/silu -> down/combine), inputs rotated over 64 activation vectors")
    res["pct_peak"] = 100.0 * res["gbs"] / PEAK_GBS
    log(f"MoE decode step ({mode}): {med:.1f} us, {res['gbs']:.0f} GB/s ({res['pct_peak']:.1f}% of 8 TB/s)")
    del ge, ue, de
    torch.cuda.empty_cache()
    return res


def bench_layer(dev, torch, steps=200, E=256, H=6144, I=2048, topk=8):
    """Next-row F2: the FFN half of a MoE decoder block at the config-2 shape -- fast RMSNorm,
    Q4_K router, 8 routed + 1 shared Q4_K SwiGLU experts, residual -- plus the RMSNorm alone
    in both modes."""
    device = "cuda"
    gen = torch.Generator(device=device)
    gen.manual_seed(98)
    ge = gen_q4k(E * I, H, gen, device)
    ue = gen_q4k(E * I, H, gen, device)
    de = gen_q4k(E * H, I, gen, device)
    rw = gen_q4k(E, H, gen, device)
    sh = (gen_q4k(I, H, gen, device), gen_q4k(I, H, gen, device), gen_q4k(H, I, gen, device))
    nx = 64
    X = (torch.randn((nx, H), device=device, generator=gen) * 0.5).to(torch.bfloat16)
    G = (1.0 + 0.1 * torch.randn(H, device=device, generator=gen)).to(torch.bfloat16)
    Y = torch.empty((nx, H), dtype=torch.bfloat16, device=device)
    ws = dev.moe_layer_workspace(E, H, I, topk, device)
    sel = torch.empty(topk, dtype=torch.int32, device=device)
    sw = torch.empty(topk, dtype=torch.bfloat16, device=device)

    def step(i):
        j = i % nx
        return lambda: dev.moe_layer_decode(Q4K, rw, Q4K, ge, ue, de, E, H, I, topk, X[j], G, mode="fast",
                                            shared=sh, workspace=ws, out=Y[j], sel_out=(sel, sw))

    ms, _ = time_graph([step(i) for i in range(steps)], reps=REPS)
    us = pct(ms, 50) * 1000.0 / steps
    res = dict(E=E, H=H, I=I, topk=topk, shared=True, router="Q4_K", us_per_step=us,
               alg_bytes=(topk + 1) * 3 * q4k_bytes(I, H) + q4k_bytes(E, H) + 4 * H * 2)
    res["gbs"] = res["alg_bytes"] / (us * 1e-6) / 1e9
    for mode in ("fast", "ref"):
        out = torch.empty(H, dtype=torch.bfloat16, device=device)
        ms, _ = time_graph([(lambda j=i: dev.rmsnorm(X[j % nx], G, mode=mode, out=out)) for i in range(200)], reps=REPS)
        res[f"rmsnorm_{mode}_us"] = pct(ms, 50) * 1000.0 / 200
    log(f"MoE layer (norm + 8+1 experts + residual): {us:.1f} us; rmsnorm fast {res['rmsnorm_fast_us']:.2f} us, "
        f"ref {res['rmsnorm_ref_us']:.2f} us")
    del ge, ue, de
    torch.cuda.empty_cache()
    return res


def bench_batched(dev, torch, steps=100, E=256, H=6144, I=2048, topk=8, Ms=(2, 4, 8)):
    """Next-row F3: the batched MoE step at the config-2 shape for M rows -- the union of the
    rows' experts evaluated once (its weights streamed once for all rows)."""
    device = "cuda"
    gen = torch.Generator(device=device)
    gen.manual_seed(97)
    ge = gen_q4k(E * I, H, gen, device)
    ue = gen_q4k(E * I, H, gen, device)
    de = gen_q4k(E * H, I, gen, device)
    rw = (torch.randn((E, H), device=device, generator=gen) * 0.05).to(torch.bfloat16)
    res = {}
    for M in Ms:
        nx = 16
        X = (torch.randn((nx, M, H), device=device, generator=gen) * 0.05).to(torch.bfloat16)
        Y = torch.empty((M, H), dtype=torch.bfloat16, device=device)
        ws = dev.moe_batched_workspace(E, H, I, topk, device)
        unions = []
        for j in range(nx):
            _, sel, _ = dev.moe_swiglu_decode_batched(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, X[j], workspace=ws,
                                                      out=Y)
            unions.append(len(set(sel.cpu().numpy().reshape(-1).tolist())))
        fns = [(lambda j=i % nx: dev.moe_swiglu_decode_batched(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, X[j],
                                                                 workspace=ws, out=Y)) for i in range(steps)]
        ms, _ = time_graph(fns, reps=REPS)
        us = pct(ms, 50) * 1000.0 / steps
        u = float(sum(unions)) / len(unions)
        alg = u * 3 * q4k_bytes(I, H) + E * H * 2 + 2 * M * H * 2
        res[f"m{M}"] = dict(M=M, us_per_step=us, us_per_row=us / M, mean_union=u, alg_bytes=alg,
                            gbs=alg / (us * 1e-6) / 1e9)
        log(f"batched MoE M={M}: {us:.1f} us ({us / M:.1f} us/row), union {u:.1f} experts, "
            f"{res[f'm{M}']['gbs']:.0f} GB/s")
    del ge, ue, de
    torch.cuda.empty_cache()
    return res


def gen_blocks(ggml_type, n_rows, K, gen, device):
    """BASELINE config-3 distributions on the device, as a flat uint8 tensor:
    Q4_K as gen_q4k; Q6_K ql/qh uniform bytes, int8 scales uniform -32..31, fp16 d = |N| 2^-8;
    Q8_0 fp16 d = |N| 2^-8 then int8 uniform -127..127; F16 N(0, 0.02)."""
    import torch
    if ggml_type == Q4K:
        return gen_q4k(n_rows, K, gen, device)
    if ggml_type == 1:
        return (torch.randn(n_rows * K, device=device, generator=gen) * 0.02).to(torch.float16).view(torch.uint8)
    if ggml_type == 14:
        nb = n_rows * K // 256
        raw = torch.randint(0, 256, (nb, 210), dtype=torch.uint8, device=device, generator=gen)
        raw[:, 192:208] = torch.randint(-32, 32, (nb, 16), dtype=torch.int8, device=device, generator=gen).view(torch.uint8)
        raw[:, 208:210] = (torch.randn(nb, device=device, generator=gen).abs() * 2.0 ** -8).to(torch.float16) \
            .view(torch.uint8).view(nb, 2)
        return raw.view(-1)
    if ggml_type == 8:
        nb = n_rows * K // 32
        raw = torch.empty((nb, 34), dtype=torch.uint8, device=device)
        raw[:, 2:34] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device, generator=gen).view(torch.uint8)
        raw[:, 0:2] = (torch.randn(nb, device=device, generator=gen).abs() * 2.0 ** -8).to(torch.float16) \
            .view(torch.uint8).view(nb, 2)
        return raw.view(-1)
    raise ValueError(ggml_type)


def bench_tiles(dev, torch, steps=200, rot_bytes=1.05e9, M=1):
    """24 column tiles of 256 rows cycling Q4_K, Q6_K, Q8_0, F16 at K=6144,
    generated on the device, for M activation rows (M > 1: a verify batch, all rows in one weight
    pass).  Cold: the launches rotate over enough distinct tile sets (>= 1 GB) that every launch
    streams its 42 MB from HBM; hot (labelled): one set, cache-resident."""
    K, rows = 6144, 256
    types = [Q4K, 14, 8, 1] * 6
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    N = rows * len(types)
    one = [gen_blocks(t, rows, K, gen, "cuda") for t in types]
    wbytes = sum(int(t.numel()) for t in one)
    nset = max(2, math.ceil(rot_bytes / wbytes))
    sets = [one] + [[gen_blocks(t, rows, K, gen, "cuda") for t in types] for _ in range(nset - 1)]
    tsets = [[(t, w, i * rows, rows) for i, (t, w) in enumerate(zip(types, ws))] for ws in sets]
    nx = 16
    xs = torch.randn((nx, M, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    nl = max(steps, nset)
    ms, _ = time_graph([(lambda j=i: dev.gemv_tiles(tsets[j % nset], N, K, xs[j % nx], mode="fast", out=y))
                        for i in range(nl)], reps=REPS)
    us = 1000.0 * pct(ms, 50) / nl
    hot_ms, _ = time_graph([(lambda j=i: dev.gemv_tiles(tsets[0], N, K, xs[j % nx], mode="fast", out=y))
                            for i in range(steps)], reps=REPS)
    hot = 1000.0 * pct(hot_ms, 50) / steps
    alg = wbytes + 2 * M * K + 2 * M * N
    del sets, tsets
    torch.cuda.empty_cache()
    log(f"mixed tiles M={M}: cold {us:.1f} us ({alg / (us * 1e-6) / 1e9:.0f} GB/s), hot {hot:.1f} us")
    return dict(N=N, K=K, M=M, us=us, alg_bytes=alg, gbs=alg / (us * 1e-6) / 1e9,
                pct_peak=100.0 * alg / (us * 1e-6) / 1e9 / PEAK_GBS, rotation_sets=nset,
                rotation_bytes=nset * wbytes, timing=f"median of {REPS} replays of one HIP graph of {nl} launches",
                hot_us_cache_resident=hot, hot_gbs_cache_resident=alg / (hot * 1e-6) / 1e9)


def bench_prefill(dev, torch, M=512, K=6144, N=16384, reps=20):
    """the matrix-core prefill GEMM (activation staging + GEMM), timed as a
    HIP graph of `reps` calls over weights rotated so that each call's weights are cold."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    wb = q4k_bytes(N, K)
    nbuf = 4
    W = gen_q4k(nbuf * N, K, gen, "cuda").view(nbuf, wb)
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = dev.prefill_workspace(M, K, "cuda")
    fns = [(lambda j=i % nbuf: dev.gemm_prefill(Q4K, W[j], N, K, x, out=y, workspace=ws)) for i in range(reps)]
    ms, _ = time_graph(fns, reps=REPS)
    t = pct(ms, 50) / reps
    fl = 2.0 * M * N * K
    del W
    torch.cuda.empty_cache()
    return dict(M=M, K=K, N=N, ms=t, tflops=fl / (t * 1e-3) / 1e12, flop=fl,
                pct_of_fp16_mfma_peak=100.0 * fl / (t * 1e-3) / 2.5e15,
                timing=f"HIP graph of {reps} calls (row scaling + operand staging + GEMM), weights rotated over {nbuf} copies")


def bench_lmhead(dev, torch, V=154880, K=6144, reps=20):
    """Next-row F4: the bf16 LM head (vocabulary x MODEL_DIM, 1.9 GB of rows, far above the
    256 MB MALL, so every call streams its weights from HBM) + argmax, bit-exact order."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8)
    w = (torch.randn((V, K), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn(K, device="cuda", generator=gen).to(torch.bfloat16)
    ws = dev.lm_head_workspace(V, "cuda")
    fns = [(lambda: dev.lm_head(w, x, workspace=ws)) for _ in range(reps)]
    ms, _ = time_graph(fns, reps=REPS)
    t = pct(ms, 50) / reps
    alg = 2 * V * K + 2 * K + 2 * V + 4
    del w
    torch.cuda.empty_cache()
    return dict(V=V, K=K, us=t * 1e3, alg_bytes=alg, gbs=alg / (t * 1e-3) / 1e9,
                pct_peak=100.0 * alg / (t * 1e-3) / 1e9 / PEAK_GBS,
                timing=f"HIP graph of {reps} calls (logits kernel + argmax pass)")


def cpu_baseline(budget_s=12.0):
    """Time the repo's CPU restatement of the reference's path on this host (1 core)."""
    import numpy as np

    from oracle import c_oracle as co
    from oracle import q4k_oracle as qo
    N = K = 6144
    rng = np.random.default_rng(42)
    raw = qo.random_q4k_blocks(rng, N * K // 256).reshape(N, -1)
    x = qo.random_bf16(rng, (1, K))
    xf = qo.bf16_bits_to_f32(x[0])
    alg = q4k_bytes(N, K) + 2 * K + 2 * N
    # (1) faithful scalar restatement (per-element np.float32 loop, as tools/q4k_ref.py)
    t0 = time.perf_counter()
    rows = 0
    while rows < 4 or time.perf_counter() - t0 < budget_s:
        r = raw[rows]
        wrow = np.concatenate([qo.dequant_block_q4k_scalar(*(lambda f: (int(f[0][0]), int(f[1][0]), f[2][0], f[3][0]))(
            qo.q4k_block_fields(r[b * 144:(b + 1) * 144]))) for b in range(K // 256)])
        qo.dot_ref_scalar(xf, wrow)
        rows += 1
        if rows >= N:
            break
    t_scalar = (time.perf_counter() - t0) / rows * N
    # (2) vectorised reference-order numpy restatement (bit-identical), full GEMV
    t0 = time.perf_counter()
    qo.gemv_quant_ref(Q4K, raw.reshape(-1), N, K, x)
    t_numpy = time.perf_counter() - t0
    # (3) plain-C restatement, single thread, full GEMV
    t0 = time.perf_counter()
    co.gemv_ref(Q4K, raw.reshape(-1), N, K, x)
    t_c = time.perf_counter() - t0
    log(f"cpu: scalar {t_scalar:.1f} s/GEMV (from {rows} rows), numpy {t_numpy:.2f} s, C {t_c:.3f} s")
    return dict(
        value=alg / t_scalar / 1e9, unit="GB/s", cores=1, kind="port",
        sample=f"faithful scalar restatement of tools/q4k_ref.py (per-element np.float32 dequant + sequential "
               f"MAC) on {rows} of 6144 rows at K=6144, extrapolated linearly in N; {N}x{K} Q4_K GEMV",
        seconds_per_gemv=t_scalar,
        numpy_vectorised=dict(value=alg / t_numpy / 1e9, unit="GB/s", cores=1, seconds_per_gemv=t_numpy),
        c_oracle=dict(value=alg / t_c / 1e9, unit="GB/s", cores=1, seconds_per_gemv=t_c),
        host_cpu_count=os.cpu_count(),
    )


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic_gemv_q4k_6144.json")
HEADLINE_KERNEL = "k_gemv1p"
COPY_BYTES = 256 << 20


def bench_copy(torch, reps=20):
    """Calibration for the HBM byte counters: a plain device copy of COPY_BYTES (torch routes a
    same-dtype contiguous copy to the runtime's copy kernel, which reads COPY_BYTES and writes
    COPY_BYTES per dispatch)."""
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return dict(bytes_read=COPY_BYTES, bytes_written=COPY_BYTES, reps=reps)


def _pmc_rows(d):
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def summarize_traffic(fetch_dir, write_dir, out=TRAFFIC_JSON):
    """HBM bytes per launch of the headline kernel from two rocprofv3 --pmc runs (FETCH_SIZE,
    then WRITE_SIZE; each over `bench.py --only gemv` followed by `--only copy`), with each
    counter scaled by what it reads for the copy kernel of known size."""
    import statistics

    def per(rows, counter, pred):
        v = [float(r["Counter_Value"]) for r in rows if r["Counter_Name"] == counter and pred(r["Kernel_Name"])]
        return statistics.median(v) if v else None

    res = {}
    for counter, d, key in (("FETCH_SIZE", fetch_dir, "bytes_read"), ("WRITE_SIZE", write_dir, "bytes_written")):
        rows = _pmc_rows(d)
        k = per(rows, counter, lambda n: HEADLINE_KERNEL in n)
        c = per(rows, counter, lambda n: "copyBuffer" in n)
        if k is None or c is None:
            raise SystemExit(f"{counter}: no samples for the headline kernel or the copy kernel in {d}")
        scale = COPY_BYTES / (c * 1024.0)     # bytes per counted KiB, from the copy of known size
        res[counter] = dict(kib_per_dispatch=k, copy_kib_per_dispatch=c, scale_bytes_per_kib=scale,
                            bytes_per_launch=k * 1024.0 * scale)
    tot = res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]
    summary = dict(kernel=HEADLINE_KERNEL, workload="Q4_K GEMV M=1 K=N=6144, cold (rotated weights)",
                   bytes_per_launch=tot, algorithmic_bytes=q4k_bytes(6144, 6144) + 4 * 6144,
                   counters=res, note="median over the dispatches of one run; calibration kernel = the runtime's "
                                      f"device copy (__amd_rocclr_copyBuffer) of {COPY_BYTES} bytes")
    with open(out, "w") as f:
        json.dump(summary, f, indent=1)
    print(json.dumps(summary))
    return summary


def _short_kernel(name):
    """`void aipu::(anonymous namespace)::k_gemv1<3, ...>(...)` -> `k_gemv1<3, ...>`."""
    n = name[5:] if name.startswith("void ") else name
    n = n.replace("aipu::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    depth, out = 0, ""
    for ch in n:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out += ch
    return out[:110]


def trace_summary(d, command):
    """Markdown summary of a `rocprofv3 --kernel-trace --stats --output-format csv` directory."""
    import csv
    import glob
    f = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no kernel_stats.csv under {d}")
    rows = list(csv.DictReader(open(f[0])))
    lines = [f"Command: `{command}`", "", "| kernel | calls | avg ns | min ns | max ns | % time |", "|---|---|---|---|---|---|"]
    for r in rows[:12]:
        lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']):.0f} | {r['MinNs']} | "
                     f"{r['MaxNs']} | {float(r['Percentage']):.1f} |")
    print("\n".join(lines))


def load_traffic():
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            return json.load(f)
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--quick", action="store_true", help="headline only, smaller rotation")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--moe-steps", type=int, default=200)
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of one HIP graph")
    ap.add_argument("--isolated", action="store_true",
                    help="with --only gemv / c0 / c1: every launch alone (host sync between launches), for kernel traces")
    ap.add_argument("--only", choices=["gemv", "moe", "stream", "copy", "tiles", "prefill", "c1", "lmhead", "layer", "batched",
                                       "floor", "c0", "exact"], default=None,
                    help="run one measurement only (for kernel tracing / counter runs)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), default=None,
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) into "
                         "profiles/traffic_gemv_q4k_6144.json and exit (no GPU needed)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("TRACE_DIR", "COMMAND"), default=None,
                    help="print a markdown table of a rocprofv3 --stats csv directory and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.traffic:
        summarize_traffic(*args.traffic)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); sharding across GPUs is "
              f"designed (rows / experts / vocabulary per GPU) but not a measured configuration.", file=sys.stderr)
        sys.exit(2)

    import torch

    from aipu_amd import device as dev
    from aipu_amd import lib
    lib()
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.init()
    rot = 0.3e9 if args.quick else 1.05e9

    if args.only == "copy":
        print(json.dumps(bench_copy(torch)))
        return
    if args.only == "moe":
        print(json.dumps(bench_moe(dev, torch, args.moe_steps)))
        return
    if args.only == "tiles":
        print(json.dumps({"m1": bench_tiles(dev, torch), "m4": bench_tiles(dev, torch, M=4)}))
        return
    if args.only == "prefill":
        print(json.dumps(bench_prefill(dev, torch)))
        return
    if args.only == "batched":
        print(json.dumps(bench_batched(dev, torch)))
        return
    if args.only == "layer":
        print(json.dumps(bench_layer(dev, torch)))
        return
    if args.only == "lmhead":
        print(json.dumps(bench_lmhead(dev, torch)))
        return
    if args.only == "c1":
        print(json.dumps({f"{mode}_m{M}": bench_gemv(dev, torch, 6144, 6144, M, 500, 20, rot, mode=mode, label="C1",
                                                     isolated=args.isolated)
                          for mode in ("fast", "fast_dense") for M in (2, 4, 8)}))
        return
    if args.only == "c0":
        print(json.dumps(bench_gemv(dev, torch, 4096, 4096, 1, 1000, 50, rot, label="C0", eager=args.eager,
                                    isolated=args.isolated)))
        return
    if args.only == "floor":
        print(json.dumps({"ns": bench_floor(dev, torch, 6144, 6144, rot), "c0": bench_floor(dev, torch, 4096, 4096, rot)}))
        return
    if args.only == "exact":
        print(json.dumps(bench_exact(dev, torch, rot)))
        return
    if args.only == "stream":
        r = bench_stream_read(dev, torch)
        r["gemv_size"] = bench_stream_read_sized(dev, torch, q4k_bytes(6144, 6144) + 4 * 6144, rot)
        print(json.dumps(r))
        return
    head = bench_gemv(dev, torch, 6144, 6144, 1, args.steps, args.warmup, rot, label="north star", eager=args.eager,
                      isolated=args.isolated and args.only == "gemv")
    if args.only == "gemv":
        print(json.dumps(head))
        return
    extra = {}
    if not args.no_extra:
        extra["stream_read_ceiling"] = bench_stream_read(dev, torch)
        log(f"stream read ceiling: {extra['stream_read_ceiling']['gbs_best']:.0f} GB/s")
        extra["stream_read_gemv_size"] = bench_stream_read_sized(dev, torch, head["alg_bytes"], rot)
        log(f"stream read of one GEMV's bytes per launch: {extra['stream_read_gemv_size']['us_per_launch']:.2f} us, "
            f"{extra['stream_read_gemv_size']['gbs']:.0f} GB/s")
        extra["moe_decode_c2"] = bench_moe(dev, torch, args.moe_steps)
        extra["gemv_c0_4096"] = bench_gemv(dev, torch, 4096, 4096, 1, 1000, 50, rot, label="C0")
        extra["floor_ns"] = bench_floor(dev, torch, 6144, 6144, rot)
        extra["floor_c0"] = bench_floor(dev, torch, 4096, 4096, rot)
        for M in (2, 4, 8):   # verify batches: rows bit-identical to the one-row launch
            extra[f"gemv_c1_m{M}"] = bench_gemv(dev, torch, 6144, 6144, M, 500, 20, rot, label="C1")
        for M in (2, 4, 8):   # opt-in dense batches: rows within the tolerance of the one-row launch
            extra[f"gemv_c1_dense_m{M}"] = bench_gemv(dev, torch, 6144, 6144, M, 500, 20, rot, mode="fast_dense",
                                                      label="C1 dense")
        extra["exact_order"] = bench_exact(dev, torch, rot)
        extra["mixed_tiles_c3"] = bench_tiles(dev, torch)
        extra["mixed_tiles_c3_m4"] = bench_tiles(dev, torch, M=4)
        extra["prefill_c4"] = bench_prefill(dev, torch)
        log(f"prefill: {extra['prefill_c4']['ms']:.2f} ms, {extra['prefill_c4']['tflops']:.1f} TFLOP/s")
        extra["lm_head_f4"] = bench_lmhead(dev, torch)
        extra["moe_layer_f2"] = bench_layer(dev, torch)
        extra["moe_batched_f3"] = bench_batched(dev, torch)
        # the bit-exact step last: run before the tile legs, it left them about 1 us slower
        # (C3 11.6 against 10.7 us when the tile legs run alone)
        extra["moe_decode_c2_ref"] = bench_moe(dev, torch, 20, mode="ref")
        log(f"lm head: {extra['lm_head_f4']['us']:.1f} us, {extra['lm_head_f4']['gbs']:.0f} GB/s")
    cpu = None if args.no_cpu else cpu_baseline()

    achieved = head["gbs"]
    out = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us_per_launch"] / 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "Q4_K GEMV M=1 K=N=6144 (north-star shape; BASELINE configs[1] at M=1)",
                   "M": 1, "K": 6144, "N": 6144, "mode": "fast", "weights": "Q4_K (ggml 144 B / 256 w)",
                   "activations": "bf16", "weight_rotation_bytes": head["weight_rotation_bytes"],
                   "timed_region": "median over 7 replays of one HIP graph of max(steps, rotation buffers) "
                                   "launches, HIP events on the replay stream around each replay"},
        "pct_of_peak": round(head["pct_peak"], 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
        "headline_detail": head,
        "extra": extra,
    }
    tr = load_traffic()
    if tr is not None:
        out["roofline"]["traffic"] = tr.get("bytes_per_launch")
        out["roofline"]["traffic_detail"] = tr
    if "moe_decode_c2" in extra:
        out["moe_decode_us"] = round(extra["moe_decode_c2"]["us_per_step"], 2)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
