#!/usr/bin/env python3
"""Benchmark of the fused int4-KV decode attention on one MI355X.

Default (the headline metric of BASELINE.json): one decode-attention layer at
Hq=32, Hkv=16, D=256, L=32768 (BASELINE configs[2] at 32k), bf16 Q, int4 K/V
with fp16 scale/bias.  A "step" is one call of ``sdpa_int4`` over one layer.
Eight distinct KV sets (8 x 151 MB) are rotated so the 256 MB Infinity Cache
cannot serve repeats; inputs are resident in HBM before timing starts.  The
calls are captured in one HIP graph of 32 launches over the sets, as a
decode step would run them, and the graph is replayed; the same launches
issued directly, back to back, are reported beside it.

Prints ONE JSON line.  Other workloads (``--workload sweep|sliding50|ragged``)
print their own line of the same shape.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0  # MI355X HBM3E, published
# HBM bytes per launch of the headline kernel, measured with rocprofv3 PMC
# counters (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, calibrated on plain copy and
# read kernels of known size); the summary file records the commands.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "sdpa_int4_mfma_ctx32k.md")


def measured_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"traffic_bytes_per_launch = .*= ([\d,]+)", line.strip())
                if m:
                    return int(m.group(1).replace(",", ""))
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--sets", type=int, default=8, help="distinct KV sets rotated")
    ap.add_argument("--workload", default="ctx32k",
                    choices=["ctx32k", "sweep", "sliding50", "ragged", "stream", "polar", "global",
                             "prefill"])
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--sb", default="f16", choices=["f16", "f32"],
                    help="K/V scale/bias dtype: f16 (BASELINE) or f32 (the reference's cache)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--out", default=None, help="also append the JSON line to this file")
    return ap.parse_args()


def gen_cache(tq, torch, Hkv, L, D, gen, cap=None, sb=None):
    """One int4 KV set built on the GPU: RMS-normed N(0,1) K, N(0,1) V,
    scale/bias in `sb` (default fp16)."""
    cap = cap or L
    sb = sb or torch.float16
    kq = torch.empty((Hkv, cap, D // 8), dtype=torch.uint32, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty((Hkv, cap, D // 64), dtype=sb, device="cuda")
    kb, vs, vb = torch.empty_like(ks), torch.empty_like(ks), torch.empty_like(ks)
    for h in range(Hkv):
        k = torch.randn((cap, D), generator=gen, device="cuda")
        k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
        v = torch.randn((cap, D), generator=gen, device="cuda")
        kq[h], ks[h], kb[h] = tq.quantize(k, scale_dtype=sb)
        vq[h], vs[h], vb[h] = tq.quantize(v, scale_dtype=sb)
    return kq, ks, kb, vq, vs, vb


def precision_note(sb_name):
    """The arithmetic of the matrix-core decode kernel, stated in full."""
    return (f"int4 K/V ({sb_name} scale/bias), bf16 Q; K.q on int8 matrix cores with q as "
            "22-bit (D 512: 21-bit) fixed point per head (exact integer dot per quant group), P.V on bf16 "
            "matrix cores with the weights p*s_v split into bf16 hi+lo (~16-bit mantissa), "
            "fp32 accumulate and softmax")


def gen_q(torch, shape, gen):
    q = torch.randn(shape, generator=gen, device="cuda")
    q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)
    return q.to(torch.bfloat16)


PREWARM_S = 0.25  # seconds of untimed steps before the warmup steps


def prewarm(torch, fn, seconds=PREWARM_S):
    """Runs fn back to back for `seconds` of wall time, untimed.  The GPU
    leaves its idle clocks only after some milliseconds under load, and a
    timed region of a few ms (100 launches of ~35 us) right after process
    start would otherwise measure part of that ramp: the same 32k layer read
    34-37 us timed first in a process and 32.4 us timed after other work."""
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(16):
            fn(i)
            i += 1
        torch.cuda.synchronize()


# Rotated input sets must exceed the 256 MB Infinity Cache (MALL) by a
# margin, or repeats are served from it: at least 512 MiB of distinct KV per
# timed workload, at most 2 GiB.
MALL_PROOF_BYTES = 512 << 20


def rotation_sets(wanted, set_bytes):
    """Number of distinct input sets to rotate: at least `wanted` and at
    least 512 MiB in all (so the MALL cannot serve a repeat), at most 2 GiB
    in all, and never fewer than 2."""
    need = -(-MALL_PROOF_BYTES // max(1, set_bytes))
    cap = (2 << 30) // max(1, set_bytes)
    return max(2, min(max(wanted, need), cap))


def time_launches(torch, fn, steps, warmup):
    """(whole-region ms per step, mean per-launch ms) with HIP events on the
    current stream -- the stream every launch is issued on.  A time-based
    pre-warm and then `warmup` untimed steps come first."""
    prewarm(torch, fn)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for i in range(steps):          # per-launch pass (kernel duration)
        ev[i][0].record()
        fn(i)
        ev[i][1].record()
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in ev)
    per_launch = sum(per) / len(per)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()                     # whole timed region, back-to-back launches
    for i in range(steps):
        fn(i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, per_launch, per[len(per) // 2]


# Sweep lengths are timed as HIP-graph replays of GRAPH_LAUNCHES launches;
# lengths above GRAPH_MAX_LEN (launches longer than one Python call) are also
# timed as direct back-to-back launches, reported beside the graph figure.
GRAPH_MAX_LEN = 8192
GRAPH_LAUNCHES = 32


def time_graph(torch, fn, n, steps, warmup):
    """time_launches of launches replayed from a graph, the way a captured
    decode step runs them (and the only way to time launches shorter than
    the host's ~10 us issue time): fn(0) .. fn(n - 1) are captured in one HIP
    graph (on a stream warmed up eagerly first, so nothing is allocated
    during capture), and the replays are timed; returns the same (ms per
    launch, mean, median) triple, per launch."""
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for i in range(n):
            fn(i)
    reps = max(1, steps // n)
    ms, mean, med = time_launches(torch, lambda i: g.replay(), reps, max(1, warmup // n))
    return ms / n, mean / n, med / n


def time_graph_and_direct(torch, fn, nsets, steps, warmup):
    """(ms per step as HIP-graph replays, ms per step issued directly, graph
    launches): fn's steps timed as replays of one graph of
    max(GRAPH_LAUNCHES, nsets) steps over the rotated sets, and as direct
    back-to-back calls."""
    ng = max(GRAPH_LAUNCHES, nsets)
    ms_graph = time_graph(torch, fn, ng, steps, warmup)[0]
    ms_direct = time_launches(torch, fn, steps, warmup)[0]
    return ms_graph, ms_direct, ng


def cpu_baseline(args, cache_host, q_host, Hq, Hkv, D, L, W, nbytes):
    """The reference algorithm (dequantize to fp32 + fp32 softmax attention)
    timed on this host with OpenMP -- oracle/tq_oracle.c (a port of the
    reference's dequantize + SDPA composition, MLX is not installed)."""
    from oracle import coracle
    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or (os.cpu_count() or 1)
    base = coracle.DequantSdpaBaseline(q_host, *cache_host, Hq // Hkv, 1.0, W, threads=threads)
    base()  # warm
    reps, t_start = 0, time.perf_counter()
    while True:
        base()
        reps += 1
        el = time.perf_counter() - t_start
        if el >= args.cpu_seconds or reps >= 200:
            break
    sec = el / reps
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "us_per_layer": round(sec * 1e6, 1),
            "sample": f"{reps} full layers (Hq={Hq} Hkv={Hkv} D={D} L={L}) of the same "
                      f"workload, dequantize->fp32 + fp32 SDPA, oracle/tq_oracle.c OpenMP, "
                      f"{platform.processor() or platform.machine()}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 "
                          "(the multi-GPU sharding of this path is a design, not built)"}))
        sys.exit(2)
    import torch
    from gemma4metal_amd import turboquant as tq
    from oracle import oracle as O

    Hq, Hkv, D = 32, 16, 256
    gen = torch.Generator(device="cuda").manual_seed(2026)
    res = {}

    sbt = torch.float32 if args.sb == "f32" else torch.float16
    sb_bytes = 4 if args.sb == "f32" else 2
    if args.workload in ("ctx32k", "sweep"):
        lens = [args.ctx] if args.workload == "ctx32k" else [1024, 8192, 32768, 131072, 262144]
        lines = []
        for L in lens:
            row = O.row_bytes(D, sb_bytes)
            nsets = rotation_sets(args.sets, Hkv * L * row)
            sets = [gen_cache(tq, torch, Hkv, L, D, gen, sb=sbt) for _ in range(nsets)]
            qs = [gen_q(torch, (Hq, D), gen) for _ in range(nsets)]
            out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
            nbytes = O.decode_bytes(Hq, Hkv, D, L, sb_bytes=sb_bytes)
            plan = tq.sdpa_plan(Hq, Hkv, D, L, sb_dtype=sbt)

            def step(i):
                s = i % nsets
                tq.sdpa_int4(qs[s], *sets[s], Hq // Hkv, 1.0, 0, out=out)

            # Replays of one HIP graph of GRAPH_LAUNCHES launches over the
            # rotated sets: the way a captured decode step issues its layers
            # (and a launch of <= 8192 keys is shorter than one Python call,
            # ~10 us to issue).  Longer launches are also timed issued
            # directly, back to back; graph replays leave less time between
            # kernels (32k: ~0.3 us per launch).
            ng = max(GRAPH_LAUNCHES, nsets)  # every rotated set in the graph
            ms_step, ms_launch, ms_med = time_graph(torch, step, ng, args.steps, args.warmup)
            timing = f"HIP graph of {ng} launches over the {nsets} sets, replayed"
            ms_direct = None
            if L > GRAPH_MAX_LEN:
                ms_direct = time_launches(torch, step, args.steps, args.warmup)[0]
            gbs = nbytes / (ms_step * 1e-3) / 1e9
            line = {
                "metric": "int4-KV decode SDPA achieved HBM GB/s at 32k ctx",
                "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
                "steps": args.steps, "warmup": args.warmup, "timing": timing,
                "ms_per_step": round(ms_step, 5), "us_per_layer": round(ms_step * 1e3, 2),
                "us_per_layer_direct_launches": (round(ms_direct * 1e3, 2)
                                                 if ms_direct is not None else None),
                "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": precision_note(args.sb),
                "data": "synthetic (seeded N(0,1), RMS-normed Q/K), random-init; "
                        f"{nsets} rotated KV sets ({nsets * Hkv * L * row / 2**20:.0f} MiB, more "
                        "than the 256 MB MALL)",
                "config": {"workload": f"sdpa_int4 decode layer Hq={Hq} Hkv={Hkv} D={D} "
                                       f"L={L} W=0, {args.sb} scale/bias (BASELINE configs[2])",
                           "global_batch": 1, "seq_len": L, "parallelism": "none (1 GPU)"},
                # the timed region is replays of launches of this one kernel
                # on one stream, so region time / launches is its mean launch
                # time
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                             "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4),
                             "kernel": plan["kernel"], "splits": plan["splits"],
                             "keys_per_split": plan["chunk"],
                             "bytes_per_launch": nbytes,
                             "us_per_launch": round(ms_step * 1e3, 2),
                             "us_per_launch_event_bracketed_mean": round(ms_launch * 1e3, 2),
                             "us_per_launch_event_bracketed_median": round(ms_med * 1e3, 2)},
            }
            # HBM bytes per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE
            # passes committed for this exact launch (headline shape, fp16
            # scale/bias); not measured by this run
            traffic = measured_traffic() if (L == 32768 and args.sb == "f16") else None
            line["roofline"]["traffic"] = traffic
            if traffic is not None:
                line["roofline"]["traffic_source"] = os.path.relpath(TRAFFIC_FILE, ROOT)
            if not args.no_cpu and L == lens[0]:
                s0 = sets[0]
                host = []
                for t in s0:
                    if t.dtype == torch.uint32:
                        host.append(t.view(torch.int32).cpu().numpy().view("uint32"))
                    else:
                        host.append(t.float().cpu().numpy())
                qh = qs[0].float().cpu().numpy()
                line["cpu_baseline"] = cpu_baseline(args, host, qh, Hq, Hkv, D, L, 0, nbytes)
            lines.append(line)
            del sets
            torch.cuda.empty_cache()
        for line in lines:
            emit(line, args)
        return

    if args.workload == "stream":
        bench_stream(args, torch, tq, O, gen, Hq, Hkv, D)
        return

    if args.workload == "polar":
        bench_polar(args, torch, gen)
        return

    if args.workload == "prefill":
        # chunked prefill through the engine's fallback attention
        # (engine/gemma4_multilayer.cpp:343-364): n_new queries after n_prior
        # cached positions, the new rows already appended
        prior, S = 3584, 512
        for label, Hq_, Hkv_, D_, W in (("sliding layer", 32, 16, 256, 1024),
                                         ("global layer", 32, 4, 512, 0)):
            L = prior + S
            cache = gen_cache(tq, torch, Hkv_, L, D_, gen, sb=sbt)
            q = gen_q(torch, (S, Hq_, D_), gen)
            out = torch.empty((S, Hq_, D_), dtype=torch.float32, device="cuda")
            plan = tq.sdpa_plan(Hq_, Hkv_, D_, L, mode="prefill", batch=S, sliding_window=W,
                                sb_dtype=sbt)
            ms, _, _ = time_launches(torch, lambda i: tq.sdpa_int4_prefill(
                q, *cache, prior, Hq_ // Hkv_, 1.0, W, out=out), args.steps, args.warmup)
            keys = sum(min(prior + i + 1, W) if W else prior + i + 1 for i in range(S))
            tflops = 4.0 * keys * D_ * Hq_ / (ms * 1e-3) / 1e12   # q.k and p.v, 2 flops per MAC
            emit({"metric": f"int4-KV prefill attention TFLOP/s, {label}",
                  "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": round(ms, 5),
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                  "dtype": (f"int4 K/V ({args.sb} scale/bias), bf16 Q; K dequantized to fp16 hi+lo "
                            "(q.k as three fp16 matrix-core products, ~22-bit), V and P as bf16 "
                            "hi+lo, fp32 accumulate"),
                  "data": "synthetic", "kernel": plan["kernel"],
                  "config": {"workload": f"prefill n_new={S} n_prior={prior} Hq={Hq_} Hkv={Hkv_} "
                                         f"D={D_} W={W}, {args.sb} scale/bias", "global_batch": 1,
                             "seq_len": L, "parallelism": "none (1 GPU)"}}, args)
        return

    if args.workload == "global":
        # Gemma global-attention layer shape (engine/gemma4_multilayer.cpp:3,49-51):
        # Hq 32, Hkv 4 (GQA 8), D 512, no window
        Hg, Hkvg, Dg, L = 32, 4, 512, args.ctx
        nsets = rotation_sets(args.sets, Hkvg * L * O.row_bytes(Dg, sb_bytes))
        sets = [gen_cache(tq, torch, Hkvg, L, Dg, gen, sb=sbt) for _ in range(nsets)]
        qs = [gen_q(torch, (Hg, Dg), gen) for _ in range(nsets)]
        out = torch.empty((Hg, Dg), dtype=torch.float32, device="cuda")
        nbytes = O.decode_bytes(Hg, Hkvg, Dg, L, sb_bytes=sb_bytes)
        plan = tq.sdpa_plan(Hg, Hkvg, Dg, L, sb_dtype=sbt)
        ms_step, ms_direct, ng = time_graph_and_direct(torch, lambda i: tq.sdpa_int4(
            qs[i % nsets], *sets[i % nsets], Hg // Hkvg, 1.0, 0, out=out), nsets, args.steps,
            args.warmup)
        gbs = nbytes / (ms_step * 1e-3) / 1e9
        emit({"metric": "int4-KV decode SDPA GB/s, Gemma global layer (D 512, GQA 8)",
              "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
              "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
              "us_per_layer": round(ms_step * 1e3, 2), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
              "timing": f"HIP graph of {ng} layers (attention + merge launches) over the "
                        f"{nsets} sets, replayed",
              "us_per_layer_direct_launches": round(ms_direct * 1e3, 2),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "dtype": precision_note(args.sb),
              "data": (f"synthetic; {nsets} rotated KV sets "
                       f"({nsets * Hkvg * L * O.row_bytes(Dg, sb_bytes) / 2**20:.0f} MiB, more than "
                       "the 256 MB MALL)"),
              "kernel": plan["kernel"], "splits": plan["splits"],
              "config": {"workload": f"sdpa_int4 Hq={Hg} Hkv={Hkvg} D={Dg} L={L} W=0, {args.sb} "
                                     "scale/bias (global layer)",
                         "global_batch": 1, "seq_len": L, "parallelism": "none (1 GPU)"}}, args)
        return

    if args.workload == "sliding50":
        L, W, layers = 786, 1024, 50
        # distinct 50-layer steps (one HIP graph each), rotated so that the
        # KV read by consecutive steps exceeds the MALL
        layer_bytes = Hkv * L * O.row_bytes(D, sb_bytes)
        nsteps = rotation_sets(1, layers * layer_bytes)
        steps_kv = [[gen_cache(tq, torch, Hkv, L, D, gen, sb=sbt) for _ in range(layers)]
                    for _ in range(nsteps)]
        q = gen_q(torch, (Hq, D), gen)
        out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
        nbytes = O.decode_bytes(Hq, Hkv, D, L, sb_bytes=sb_bytes)

        def one_step(sets):
            for s in sets:
                tq.sdpa_int4(q, *s, Hq // Hkv, 1.0, W, out=out)
        # warm the capture stream up eagerly, so its split-K workspace exists
        # before capture (nothing is allocated inside the graphs)
        cs = torch.cuda.Stream()
        with torch.cuda.stream(cs):
            one_step(steps_kv[0])
        torch.cuda.synchronize()
        graphs = []
        for sets in steps_kv:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                one_step(sets)
            graphs.append(g)
        ms_step, ms_launch, _ = time_launches(torch, lambda i: graphs[i % nsteps].replay(),
                                              args.steps, args.warmup)
        us_layer = ms_step * 1e3 / layers
        gbs = nbytes * layers / (ms_step * 1e-3) / 1e9
        emit({"metric": "int4-KV decode SDPA, 50 sliding layers (HIP graph) GB/s",
              "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
              "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
              "us_per_layer": round(us_layer, 3), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "dtype": precision_note(args.sb),
              "data": f"synthetic; {nsteps} distinct 50-layer KV sets rotated "
                      f"({nsteps * layers * layer_bytes / 2**20:.0f} MiB, more than the 256 MB MALL)",
              "config": {"workload": "50 x sdpa_int4 Hq=32 Hkv=16 D=256 L=786 W=1024, "
                                     f"{args.sb} scale/bias (BASELINE configs[1]), one HIP graph "
                                     "per step",
                         "global_batch": 1, "seq_len": L, "parallelism": "none (1 GPU)"}},
             args)
        return

    if args.workload == "ragged":
        import numpy as np
        B, cap = 64, 32768 + 1
        rng = np.random.default_rng(4)
        lens = rng.integers(512, 32768, size=B, endpoint=True).astype(np.int32)
        wins = np.array([1024 if b % 2 == 0 else 0 for b in range(B)], np.int32)
        cache = tq.Int4KVCache(B, Hkv, cap, D, "cuda")
        for b in range(B):
            c = gen_cache(tq, torch, Hkv, int(lens[b]), D, gen, cap=int(lens[b]))
            for dst, src in zip(cache.tensors(), c):
                dst[b, :, :int(lens[b])] = src
        lens_d = torch.from_numpy(lens).cuda()
        wins_d = torch.from_numpy(wins).cuda()
        q = gen_q(torch, (B, Hq, D), gen)
        knew = torch.randn((B, Hkv, 1, D), generator=gen, device="cuda")
        vnew = torch.randn((B, Hkv, 1, D), generator=gen, device="cuda")
        out = torch.empty((B, Hq, D), dtype=torch.float32, device="cuda")
        attended = int(sum(min(int(l) + 1, int(w)) if w else int(l) + 1
                           for l, w in zip(lens, wins)))
        nbytes = (Hkv * attended * 288 + B * Hq * D * 6 + 2 * B * Hkv * D * 4
                  + 2 * B * Hkv * 144)

        def step(i):
            cache.lengths.copy_(lens_d)
            cache.append(knew, vnew)
            tq.sdpa_int4_ragged(q, *cache.tensors(), cache.lengths, Hq // Hkv, 1.0, 0,
                                windows=wins_d, max_kv_len=cap, out=out)
        ms_step, ms_launch, _ = time_launches(torch, step, args.steps, args.warmup)
        gbs = nbytes / (ms_step * 1e-3) / 1e9
        emit({"metric": "int4-KV ragged batched decode + append GB/s", "value": round(gbs, 1),
              "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "ms_per_step": round(ms_step, 5), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "dtype": "int4 K/V (fp16 scale/bias), bf16 Q", "data": "synthetic",
              "config": {"workload": "B=64 ragged L~U[512,32768] (seed 4), W=1024 on even b, "
                                     "append 1 fp32 token/seq then decode (BASELINE configs[3])",
                         "global_batch": B, "seq_len": cap, "parallelism": "none (1 GPU)",
                         "algorithmic_bytes": nbytes}}, args)
        return


def bench_stream(args, torch, tq, O, gen, Hq, Hkv, D):
    """Achievable-bandwidth ceiling of the headline launch.  Plain streaming
    reads over exactly the headline's algorithmic bytes (151,044,096 B),
    rotating over disjoint windows of a 1 GiB buffer so the 256 MB MALL
    serves no repeat: the grid-stride read, and the tiled read in the
    attention kernel's own geometry (one workgroup per CU over a contiguous
    slice, 8 waves, 16-byte loads, iterations in flight) over a sweep of
    loads per lane, pipeline depth and load policy.  The attention launch is
    timed in the same process, so kernel / ceiling is a same-box ratio."""
    import ctypes
    from gemma4metal_amd import _lib
    nbytes = 1 << 30
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").normal_()
    bdst = torch.empty_like(a)
    ms_copy, _, _ = time_launches(torch, lambda i: bdst.copy_(a), args.steps, args.warmup)
    del bdst
    acc = torch.empty((), dtype=torch.float32, device="cuda")
    ms_sum, _, _ = time_launches(torch, lambda i: torch.sum(a, dim=0, out=acc), args.steps,
                                 args.warmup)
    copy_gbs = 2 * nbytes / (ms_copy * 1e-3) / 1e9
    read_gbs = nbytes / (ms_sum * 1e-3) / 1e9
    sink = torch.empty(65536 * 256, dtype=torch.int32, device="cuda")
    hl = O.decode_bytes(Hq, Hkv, D, 32768)  # 151,044,096
    nwin = nbytes // hl

    def sptr():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    grid_stride = {}
    for blocks in (1024, 2048, 4096):
        ms_p, _, _ = time_launches(torch, lambda i: _lib.call(
            "tq_stream_read", ctypes.c_void_p(a.data_ptr() + (i % nwin) * hl), hl,
            ctypes.c_void_p(sink.data_ptr()), blocks, sptr()), args.steps, args.warmup)
        grid_stride[blocks] = round(ms_p * 1e3, 2)
    tiles = []
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    for waves, u, depth, nt, blocks in (
            (8, 9, 1, 1, ncu), (8, 9, 1, 0, ncu), (8, 9, 2, 1, ncu), (8, 9, 2, 0, ncu),
            (8, 4, 1, 1, ncu), (8, 4, 2, 1, ncu), (8, 4, 3, 1, ncu), (8, 16, 1, 1, ncu),
            (4, 16, 1, 1, ncu), (4, 9, 2, 1, ncu), (16, 4, 1, 1, ncu), (16, 4, 2, 1, ncu),
            (16, 9, 1, 1, ncu), (8, 9, 1, 1, 2 * ncu), (8, 4, 2, 1, 2 * ncu),
            (8, 4, 3, 0, ncu)):
        ms_p, _, _ = time_launches(torch, lambda i: _lib.call(
            "tq_stream_read_tiles", ctypes.c_void_p(a.data_ptr() + (i % nwin) * hl), hl,
            ctypes.c_void_p(sink.data_ptr()), blocks, waves, u, depth, nt, sptr()),
            args.steps, args.warmup)
        tiles.append({"waves": waves, "loads_per_lane": u, "depth": depth, "nt": nt,
                      "blocks": blocks, "us": round(ms_p * 1e3, 2),
                      "gbs": round(hl / (ms_p * 1e-3) / 1e9, 1)})
    # the floor at the sliding layer's size (configs[1], 16 x 786 x 288 B):
    # one workgroup per kv head (a single pass, no split merge) up to the
    # planner's split counts and beyond.  A launch this short is shorter
    # than a Python call, so 50 launches (rotated windows) are one HIP
    # graph, as in the sliding50 workload, and a launch is a replay / 50.
    small = Hkv * 786 * 288
    nwin_s = nbytes // (small + 4096)
    small_floor = []
    for blocks in (Hkv, 2 * Hkv, 4 * Hkv, 7 * Hkv, ncu):
        for waves, u, depth in ((8, 4, 1), (8, 4, 3), (8, 9, 2), (8, 16, 1), (16, 4, 3), (16, 9, 1)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(50):
                    _lib.call("tq_stream_read_tiles",
                              ctypes.c_void_p(a.data_ptr() + (i % nwin_s) * (small + 4096)), small,
                              ctypes.c_void_p(sink.data_ptr()), blocks, waves, u, depth, 1, sptr())
            ms_p, _, _ = time_launches(torch, lambda i: g.replay(), max(5, args.steps // 50),
                                       max(2, args.warmup // 50))
            del g
            small_floor.append({"blocks": blocks, "waves": waves, "loads_per_lane": u, "depth": depth,
                                "us": round(ms_p * 1e3 / 50, 2)})
    del a
    torch.cuda.empty_cache()
    # the attention launch itself, same box, same rotation rule
    L = 32768
    nsets = max(2, min(args.sets, (2 << 30) // max(1, Hkv * L * 288)))
    sets = [gen_cache(tq, torch, Hkv, L, D, gen) for _ in range(nsets)]
    qs = [gen_q(torch, (Hq, D), gen) for _ in range(nsets)]
    out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
    ms_attn, _, _ = time_launches(torch, lambda i: tq.sdpa_int4(
        qs[i % nsets], *sets[i % nsets], Hq // Hkv, 1.0, 0, out=out), args.steps, args.warmup)
    best = min(tiles, key=lambda t: t["us"])
    emit({"metric": "achievable HBM streaming read of the headline's 151,044,096 B (one launch)",
          "value": best["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
          "warmup": args.warmup, "ms_per_step": round(best["us"] * 1e-3, 5),
          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
          "data": "synthetic", "best_tiled": best, "tiled_sweep": tiles,
          "grid_stride_us_by_blocks": grid_stride,
          "attention_us_same_box": round(ms_attn * 1e3, 2),
          "attention_over_best_probe": round(ms_attn * 1e3 / best["us"], 4),
          "torch_sum_1GiB_gbs": round(read_gbs, 1), "torch_copy_1GiB_gbs": round(copy_gbs, 1),
          "sliding_layer_bytes": small, "sliding_layer_sweep": small_floor,
          "config": {"workload": "streaming read probes over 151,044,096 B, rotated windows",
                     "global_batch": 1, "seq_len": 32768, "parallelism": "none (1 GPU)"}}, args)


def bench_polar(args, torch, gen):
    """PolarQuant (7 levels) + QJL keys and int4 V at
    Hq=32, Hkv=16, D=128, L=32768, N(0,1) keys and query, attn_scale 1.0.
    A step = one attention launch straight from q (each workgroup builds its
    heads' query tables: q' = P q, S q'); beside it are timed the two-launch
    form (query preparation, then attention over the prepared tables), the
    attention launch alone, and the score-only launch."""
    from gemma4metal_amd import polar as pq
    from gemma4metal_amd import turboquant as tq
    from oracle import polar as PQ
    Hq, Hkv, D, L = 32, 16, 128, 32768
    P = torch.linalg.qr(torch.randn((D, D), generator=gen, device="cuda", dtype=torch.float64))[0]
    P = P.to(torch.float32).contiguous()
    S = torch.randn((128, D), generator=gen, device="cuda")
    codec = pq.Polar7Codec(P, S)
    nsets = rotation_sets(args.sets, Hkv * L * 140)  # 140 B per (kv head, key)
    sets = []
    for _ in range(nsets):
        k = torch.randn((Hkv, L, D), generator=gen, device="cuda")
        v = torch.randn((Hkv, L, D), generator=gen, device="cuda")
        keys = codec.encode(k)
        vals = tq.quantize(v, scale_dtype=torch.float16)
        sets.append((keys, vals))
        del k, v
    qs_ = [torch.randn((Hq, D), generator=gen, device="cuda") for _ in range(nsets)]
    out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
    nbytes = PQ.polar7_decode_bytes(Hq, Hkv, L)
    prepared = [codec.prepare_query(q) for q in qs_]

    def step(i):
        s = i % nsets
        codec.sdpa_int4v_q(qs_[s], *sets[s][0], *sets[s][1], 1.0, 0, out=out)

    def two_launch(i):
        s = i % nsets
        tab = codec.prepare_query(qs_[s])
        codec.sdpa_int4v(tab, *sets[s][0], *sets[s][1], 1.0, 0, out=out)

    def attn_only(i):
        s = i % nsets
        codec.sdpa_int4v(prepared[s], *sets[s][0], *sets[s][1], 1.0, 0, out=out)

    def score_only(i):
        s = i % nsets
        codec.score(prepared[s], *sets[s][0])

    def score_q(i):
        s = i % nsets
        codec.score_q(qs_[s], *sets[s][0])

    ms_step, ms_step_direct, ng = time_graph_and_direct(torch, step, nsets, args.steps, args.warmup)
    ms_two = time_graph_and_direct(torch, two_launch, nsets, args.steps, args.warmup)[0]
    ms_attn = time_graph_and_direct(torch, attn_only, nsets, args.steps, args.warmup)[0]
    ms_score = time_graph_and_direct(torch, score_only, nsets, args.steps, args.warmup)[0]
    ms_score_q = time_graph_and_direct(torch, score_q, nsets, args.steps, args.warmup)[0]
    score_bytes = Hkv * L * 68 + 2 * Hq * D * 4 + Hq * L * 4
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    gbs_attn = nbytes / (ms_attn * 1e-3) / 1e9
    emit({"metric": "PolarQuant+QJL compressed-key decode attention GB/s at 32k ctx",
          "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
          "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
          "us_per_layer": round(ms_step * 1e3, 2), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
          "timing": f"HIP graph of {ng} steps over the {nsets} sets, replayed (every form below "
                    "too)",
          "us_per_layer_direct_launches": round(ms_step_direct * 1e3, 2),
          "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
          "dtype": "polar7 angles + 128-bit QJL sketch (fp16 norms), int4 V (fp16 scale/bias), "
                   "f32 q, f32 accumulate",
          "data": f"synthetic (seeded N(0,1) K/V/q, seeded orthogonal P and N(0,1) S); "
                  f"{nsets} rotated KV sets ({nsets * Hkv * L * 140 / 2**20:.0f} MiB, more than the "
                  f"256 MB MALL)",
          "config": {"workload": f"polar7+QJL decode layer Hq={Hq} Hkv={Hkv} D={D} L={L} "
                                 "(BASELINE configs[4])", "global_batch": 1, "seq_len": L,
                     "parallelism": "none (1 GPU)"},
          "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                       "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                       "kernel": "polar7_sdpa_kernel<2,__half,8,true> (query tables built in-kernel)",
                       "bytes_per_launch": nbytes, "us_per_launch": round(ms_step * 1e3, 2)},
          "two_launch": {"us_per_step": round(ms_two * 1e3, 2),
                         "attention_us_per_launch": round(ms_attn * 1e3, 2),
                         "attention_gbs": round(gbs_attn, 1)},
          "score_only": {"us_per_launch": round(ms_score * 1e3, 2), "bytes_per_launch": score_bytes,
                         "gbs": round(score_bytes / (ms_score * 1e-3) / 1e9, 1),
                         "from_q_us_per_launch": round(ms_score_q * 1e3, 2)}}, args)


def emit(line, args):
    s = json.dumps(line)
    print(s, flush=True)
    if args.out:
        with open(args.out, "a") as f:
            f.write(s + "\n")


if __name__ == "__main__":
    main()
