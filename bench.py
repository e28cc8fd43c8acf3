"""Benchmark of the MI355X attention hot path: the headline metric (decode-attention µs per layer and achieved HBM
GB/s) on its peak-load config.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3] [--no-cpu-baseline]

A step is one decode tick of the slow AR's attention: 24 layers x (bias_rope_store -> split-K decode
attention) over 192 slots at KV length 2048 (config 3), captured once as a HIP graph and replayed. Inputs
(per-layer fused qkv rows, biases, 24 distinct layer caches = 4.5 GiB, so no layer's KV is served from the
256 MB MALL on the next replay) are resident in HBM before the timed region.

Prints ONE JSON line: value = algorithmic HBM bytes of the tick / tick time (GB/s), plus µs per layer, the
roofline of the dominant kernel (the decode kernel, timed live with HIP events on its stream over a graph of
24 decode launches) and the CPU baseline (the CPU oracle on a bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/layer + achieved HBM GB/s (% peak) at 192 slots, KV 2048"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFLOPS = 2500.0
NQ, NKV, HD, LAYERS = 14, 2, 64, 24
W = (NQ + 2 * NKV) * HD


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="C3", choices=["C2", "C3"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU-baseline sample")
    p.add_argument("--shape", default=None, help="use the split + combine kernels at NSPLIT,WAVES")
    p.add_argument("--stream-shape", default=None, help="force the streaming kernel's WAVES,TILES_PER_WAVE,GRID")
    p.add_argument("--no-configs", action="store_true", help="skip the other configs' figures (C1, C2, C4, C5)")
    p.add_argument("--traffic-probe", action="store_true",
                   help="only launch one layer's decode 4x and a 256 MiB copy (target of rocprofv3 --pmc passes)")
    p.add_argument("--prefill-probe", action="store_true",
                   help="only launch the C4 prefill 3x (target of rocprofv3 --pmc passes)")
    p.add_argument("--vocoder-probe", action="store_true",
                   help="only run the streaming decoder for 5 frames at 192 rows (target of rocprofv3)")
    p.add_argument("--slow-probe", action="store_true",
                   help="only tune GemmDispatch and replay the 24-layer slow-AR step 3 times (target of rocprofv3)")
    p.add_argument("--gemm-shapes", default=None,
                   help="with --slow-probe: these gemm_small shapes (NxK:splits:mblocks,...) instead of the tuned ones "
                        "(the tuning's timings under a profiler differ from the bench's)")
    return p.parse_args()


def build_workload(a8, torch, cfg, dev, seed=0):
    """Per-layer inputs and caches of config 3 (or config 2) on the device."""
    g = torch.Generator(device=dev).manual_seed(seed)
    if cfg == "C3":
        b, S = 192, 2048
        lens = torch.full((b,), 2048, dtype=torch.int32)
    else:
        b, S = 64, 4096
        lens = torch.randint(128, 2049, (b,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    st = a8.AttnStack(LAYERS, NQ, NKV, HD, 10000.0, max_rows=max(16 * b, 8192), cache_rows=b + 1, cache_len=S,
                      max_pos=S, dev=dev)
    for i in range(LAYERS):
        st.kc[i].normal_(generator=g)
        st.vc[i].normal_(generator=g)
    pos = (lens - 1).to(dev)
    slot = torch.arange(b, dtype=torch.int32, device=dev)
    qkv = [torch.randn(b, W, generator=g, device=dev).to(torch.bfloat16) for _ in range(LAYERS)]
    bias = [(torch.randn(W, generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(LAYERS)]
    q = torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev) for _ in range(LAYERS)]
    return dict(st=st, b=b, S=S, lens_h=lens, lens=lens.to(dev), pos=pos, slot=slot, qkv=qkv, bias=bias, q=q,
                outs=outs)


def capture(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_median(torch, g, steps, warmup, runs=5):
    """Median over `runs` of time_graph (ms per replay)."""
    return statistics.median(time_graph(torch, g, steps, warmup if i == 0 else 2) for i in range(runs))


def time_graph(torch, g, steps, warmup):
    """ms per replay: warmup replays, then `steps` replays between two events on the launching stream."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def host_cpu():
    """(model name, logical CPUs the OS reports) of this host, from /proc/cpuinfo (lscpu's source)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, os.cpu_count()


def cpu_baseline(w, budget_s):
    """The CPU oracle (torch on the host cores) on one layer of the same workload: store + decode for all
    slots, repeated until the budget is spent (at least 3 reps); median per layer. Threads: torch's intra-op
    pool as the process starts it (OMP_NUM_THREADS when set: on the GPU boxes that is the share of cores a
    one-GPU job gets, which may be fewer than os.cpu_count() reports); both counts are recorded."""
    import torch
    from oracle import attn_ref as ref

    threads = torch.get_num_threads()
    st = w["st"]
    b, S = w["b"], w["S"]
    kc, vc = st.kc[0].cpu(), st.vc[0].cpu()
    qkv, bias = w["qkv"][0].cpu(), w["bias"][0].cpu()
    pos, slot, lens = w["pos"].cpu(), w["slot"].cpu(), w["lens"].cpu()
    cos, sin = ref.rope_tables(10000.0, HD, S)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 200):
        q = torch.empty(b, NQ, HD, dtype=torch.bfloat16)
        t0 = time.perf_counter()
        ref.bias_rope_store(qkv, bias, cos, sin, pos, slot, q, kc, vc, NQ, NKV, HD)
        ref.decode_attention(q, kc, vc, lens, nsplit=1)
        times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times)
    nbytes = ref.decode_bytes(w["lens_h"].tolist(), NQ, NKV, HD)
    model, ncpu = host_cpu()
    return {"value": round(nbytes / per_layer / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "us_per_layer": round(per_layer * 1e6, 1), "cpu_model": model, "os_cpu_count": ncpu,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "sample": f"1 of {LAYERS} layers (store + decode, {b} slots, same inputs), {len(times)} reps, median"}


def cpu_leg(fn, work, unit, budget_s, sample):
    """The CPU oracle timed on the host cores (torch's intra-op threads): fn() repeated until budget_s is spent
    (at least one rep, at least three when they are short), median. work: bytes (GB/s) or FLOPs (GFLOP/s) per
    call."""
    import torch
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (len(times) < 3 and times[0] < budget_s / 3) or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    model, ncpu = host_cpu()
    return {"value": round(work / med / 1e9, 3), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "us_per_call": round(med * 1e6, 1), "cpu_model": model, "os_cpu_count": ncpu, "reps": len(times),
            "sample": sample}


BUCKETS = (1, 8, 16, 32, 64, 96, 128, 144, 160, 176, 192)


def bucket_sweep(a8, torch, w, steps):
    """The peak-load tick at every tick bucket of the reference (fast_engine.py:669-670: one graph per bucket
    up to 192 slots, each with its own split count, 776): the first b slots of the C3 workload at KV 2048, 24
    layers of the fused store + decode as one graph, the reference's split count passed as the lower bound.
    µs per layer, GB/s and the fraction of HBM peak per bucket, with the schedule the call takes."""
    from oracle import attn_ref as ref_counts  # byte counts only
    st = w["st"]
    res = {}
    for b in BUCKETS:
        qkv = [x[:b] for x in w["qkv"]]
        outs = [o[:b] for o in w["outs"]]
        nsplit = a8.ref_nsplit(b, NKV)
        g = capture(torch, lambda: st.forward(qkv, w["bias"], w["pos"][:b], w["slot"][:b], w["lens"][:b],
                                              nsplit=nsplit, rowmap=False, q=w["q"][:b], outs=outs, fuse=True))
        us = time_median(torch, g, steps, 10) * 1e3 / LAYERS
        del g
        nbytes = ref_counts.decode_bytes(w["lens_h"][:b].tolist(), NQ, NKV, HD)
        kind, shape = st.attn.schedule(b, w["S"], nsplit, fused=True)
        res[str(b)] = {"us_per_layer": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                       "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "schedule": [kind, list(shape)]}
    return res


def per_config(a8, torch, dev, steps, cpu_budget=4.0):
    """µs per layer (per pass at C5), achieved GB/s or TFLOP/s and the roofline fraction of the other benchmark
    configs, each timed as a captured graph (median of 5 runs). Decode configs: store + decode per layer, the
    engine's calls (fused where the schedule allows). C4: store + packed prefill per layer, and the prefill
    launch alone against the bf16 MFMA peak. With cpu_budget > 0, C1, C2, C4 and C5 also carry the CPU
    oracle (the reference's semantics in torch on the host cores) timed on one layer / pass of the same inputs."""
    from oracle import attn_ref as ref_counts  # byte / FLOP counts and the CPU-baseline legs
    import numpy as np

    res = {}
    gen = torch.Generator(device=dev).manual_seed(7)

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(torch.bfloat16)

    # C1: one row, KV 385 after storing position 384; C2: 64 slots, lengths U[128, 2048], cache 4096
    for cfg in ("C1", "C2"):
        if cfg == "C1":
            b, S, layers = 1, 512, LAYERS
            lens = torch.full((b,), 385, dtype=torch.int32)
        else:
            b, S, layers = 64, 4096, LAYERS
            lens = torch.randint(128, 2049, (b,), generator=torch.Generator().manual_seed(0), dtype=torch.int32)
        st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=max(16 * b, 8192), cache_rows=b + 1, cache_len=S,
                          max_pos=S, dev=dev)
        for i in range(layers):
            st.kc[i].normal_(generator=gen)
            st.vc[i].normal_(generator=gen)
        lens_d, pos, slot = lens.to(dev), (lens - 1).to(dev), torch.arange(b, dtype=torch.int32, device=dev)
        qkv = [randn(b, W) for _ in range(layers)]
        bias = [randn(W, std=0.02) for _ in range(layers)]
        q = torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev)
        outs = [torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
        nsplit = a8.ref_nsplit(b, NKV)
        g = capture(torch, lambda: st.forward(qkv, bias, pos, slot, lens_d, nsplit=nsplit, rowmap=False, q=q,
                                              outs=outs, fuse=True))
        us = time_median(torch, g, steps, 10) * 1e3 / layers
        nbytes = ref_counts.decode_bytes(lens.tolist(), NQ, NKV, HD)
        kind, shape = st.attn.schedule(b, S, nsplit, fused=True)
        res[cfg] = {"us_per_layer": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                    "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes,
                    "schedule": [kind, list(shape)], "rows": b, "kv_len": int(max(lens)),
                    "note": "latency bound" if cfg == "C1" else "store + decode per layer"}
        if cpu_budget > 0:  # the CPU oracle on layer 0's inputs: store, then decode (C1: its whole layer)
            kc_h, vc_h = st.kc[0].cpu(), st.vc[0].cpu()
            qkv_h, bias_h, pos_h, slot_h = qkv[0].cpu(), bias[0].cpu(), pos.cpu(), slot.cpu()
            cos_h, sin_h = ref_counts.rope_tables(10000.0, HD, S)

            def cpu_layer():
                qh = torch.empty(b, NQ, HD, dtype=torch.bfloat16)
                ref_counts.bias_rope_store(qkv_h, bias_h, cos_h, sin_h, pos_h, slot_h, qh, kc_h, vc_h, NQ, NKV, HD)
                ref_counts.decode_attention(qh, kc_h, vc_h, lens, nsplit=1)

            res[cfg]["cpu_baseline"] = cpu_leg(cpu_layer, nbytes, "GB/s", cpu_budget,
                                               f"1 of {layers} layers (store + decode, {b} rows, same inputs)")
        del g, st, qkv, outs
        torch.cuda.empty_cache()

    # C5: fast-AR shape, 192 slots x 4 layers, cache [192, 2, 10, 64]: a 2-token pass (384 rows at positions
    # 0 / 1 sharing their slot, rowmap = slot) then 8 passes of 192 rows at positions 2..9
    b, S, layers = 192, 10, 4
    st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=max(2 * 2 * b, 16), cache_rows=b, cache_len=S,
                      max_pos=16, dev=dev, nsplit_max=1)
    passes = []
    r = torch.arange(2 * b, dtype=torch.int32)
    passes.append(((r % 2).to(dev), (r // 2).to(dev), (r % 2 + 1).to(dev), True, 2 * b))
    for p in range(2, 10):
        rows = torch.arange(b, dtype=torch.int32)
        passes.append((torch.full((b,), p, dtype=torch.int32, device=dev), rows.to(dev),
                       torch.full((b,), p + 1, dtype=torch.int32, device=dev), False, b))
    qkvs = [[randn(nr, W) for _ in range(layers)] for (_, _, _, _, nr) in passes]
    bias = [randn(W, std=0.02) for _ in range(layers)]
    q = torch.empty(2 * b, NQ, HD, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(2 * b, NQ, HD, dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    def c5():
        # the 2-token pass stores two rows per slot and must store before it attends; the later passes have
        # one row per slot and no row map (fast_engine.py:710), so they store and attend in one launch
        for (pos, slot, lens_d, rmap, nr), qkv in zip(passes, qkvs):
            st.forward(qkv, bias, pos, slot, lens_d, nsplit=1, rowmap=rmap, q=q[:nr], outs=[o[:nr] for o in outs],
                       fuse=not rmap)

    g = capture(torch, c5)
    us = time_median(torch, g, steps, 10) * 1e3 / (len(passes) * layers)
    res["C5"] = {"us_per_pass_layer": round(us, 3), "passes": len(passes), "layers": layers, "rows": b,
                 "schedule": [list(st.attn.schedule(2 * b, S)), list(st.attn.schedule(b, S, fused=True))],
                 "note": "latency bound (<= 1 MB of KV per pass)"}
    if cpu_budget > 0:  # the CPU oracle on one pass-layer: the 192-row pass at position 5 (lens 6), layer 0
        pos5, slot5, lens5, _, nr5 = passes[4]
        kc_h, vc_h = st.kc[0].cpu(), st.vc[0].cpu()
        qkv_h, bias_h = qkvs[4][0].cpu(), bias[0].cpu()
        cos_h, sin_h = ref_counts.rope_tables(10000.0, HD, 16)
        pos_h, slot_h, lens_h = pos5.cpu(), slot5.cpu(), lens5.cpu()

        def cpu_pass():
            qh = torch.empty(nr5, NQ, HD, dtype=torch.bfloat16)
            ref_counts.bias_rope_store(qkv_h, bias_h, cos_h, sin_h, pos_h, slot_h, qh, kc_h, vc_h, NQ, NKV, HD)
            ref_counts.decode_attention(qh, kc_h, vc_h, lens_h, nsplit=1)

        res["C5"]["cpu_baseline"] = cpu_leg(cpu_pass, ref_counts.decode_bytes(lens_h.tolist(), NQ, NKV, HD), "GB/s",
                                            cpu_budget, "one pass-layer (192 rows at position 5, store + decode)")
    del g, st, qkvs, outs
    torch.cuda.empty_cache()

    # The whole slow-AR decode step (beside configs C1-C5): 24 layers x (rmsnorm, qkv GEMM, fused store + decode,
    # o GEMM, residual + rmsnorm, w13 GEMM, silu_mul, w2 GEMM, residual + rmsnorm) over 192 slots at KV 2048,
    # one graph. Synthetic weights of the slow AR's shapes (width 896; the MLP width 4864 is an assumption:
    # the checkpoint is absent offline); GEMMs are hipBLASLt through torch.matmul.
    from importlib import import_module
    ss = import_module(a8.__name__ + ".slow_stack")
    b, S, layers, hidden, inter = 192, 2048, LAYERS, 896, 4864
    wts, norm = ss.random_weights(layers, hidden, NQ, NKV, HD, inter, dev, seed=11)
    st = a8.SlowStack(wts, norm, NQ, NKV, HD, 1e-6, 10000.0, max_rows=max(16 * b, 8192), cache_rows=b + 1,
                      cache_len=S, max_pos=S, dev=dev)
    st.kc_all.normal_(generator=gen)
    st.vc_all.normal_(generator=gen)
    x0 = randn(b, hidden)
    xbuf = x0.clone()
    lens_d = torch.full((b,), S, dtype=torch.int32, device=dev)
    pos, slot = lens_d - 1, torch.arange(b, dtype=torch.int32, device=dev)
    g = capture(torch, lambda: st.forward(xbuf, pos, slot, lens_d, rowmap=False, fuse=True))
    us = time_median(torch, g, max(steps // 5, 5), 3) * 1e3
    wbytes = layers * 2 * (hidden * (NQ + 2 * NKV) * HD + hidden * NQ * HD + hidden * 2 * inter + inter * hidden)
    lib_step = {"us_per_step": round(us, 1), "us_per_layer": round(us / layers, 2),
                "note": "projections through hipBLASLt (torch.matmul, the reference's default mm), silu_mul "
                        "separate"}
    del g
    # the same step with the projections through GemmDispatch: per shape, hipBLASLt or this package's small-M
    # GEMM (gemm_small, with its split count and row blocks), whichever the timing at startup finds faster --
    # timed cycling through the 24 layers' weights, as the step reads them
    mm = a8.GemmDispatch()
    mm.tune([L[k] for L in wts for k in ("wqkv", "wo", "w13", "w2")], [b], gated=[L["w13"] for L in wts],
            large_m=8192)
    st.mm = mm
    xbuf.copy_(x0)
    g = capture(torch, lambda: st.forward(xbuf, pos, slot, lens_d, rowmap=False, fuse=True))
    us_dispatch = time_median(torch, g, max(steps // 5, 5), 3) * 1e3
    del g
    # the same step with the residual RMSNorms inside the projections (SlowStack.fuse_norm: gemm_small_norm,
    # two launches fewer per layer)
    st.fuse_norm = True
    xbuf.copy_(x0)
    g = capture(torch, lambda: st.forward(xbuf, pos, slot, lens_d, rowmap=False, fuse=True))
    us2 = time_median(torch, g, max(steps // 5, 5), 3) * 1e3
    res["slow_ar_step"] = {
        "us_per_step": round(us2, 1), "us_per_layer": round(us2 / layers, 2), "rows": b, "kv_len": S,
        "hidden": hidden, "inter": inter, "weight_bytes": wbytes,
        "choices": {f"{N}x{K}": (None if c is None else {"splits": c[0], "mblocks": c[1]})
                    for (M, N, K), c in mm.small.items()},
        "gemm_small_shapes": {f"{N}x{K}": {"splits": c[0], "mblocks": c[1]} for (M, N, K), c in mm.small_best.items()},
        "gated_shapes": {f"{N}x{K}": {"mblocks": c[1]} for (M, N, K), c in mm.gated_best.items()},
        "tune_us": {f"{N}x{K}": [None if lt is None else round(lt * 1e3, 2), None if bt is None else round(bt * 1e3, 2)]
                    for (M, N, K), lt, _, bt in mm.log},
        "prefill_sized_m": {f"{N}x{K}": v for (N, K), v in mm.large.items()},
        "library": lib_step,
        "norms_separate": {"us_per_step": round(us_dispatch, 1), "us_per_layer": round(us_dispatch / layers, 2),
                           "note": "GemmDispatch per shape (hipBLASLt or gemm_small), rmsnorm as its own launch"},
        "note": "the full slow-AR decode step around the attention path (fused store + decode, the four "
                "projections, the residual RMSNorms, SiLU-mul); synthetic weights; projections on gemm_small "
                "(its fastest shape per weight, timed at startup on the layers' weights) with the norms inside "
                "them (SlowStack.fuse_norm: the o / w2 products add the residual and leave the norm's sums of "
                "squares, the qkv / w13 products apply it, w13 with SiLU-mul in its epilogue). Numerics: the "
                "reference rounds rmsnorm's output to bf16 (twice) before each product; the fused products "
                "scale their fp32 sums by 1 / rms and round the weight folded with the norm weight instead "
                "(within bf16 noise of the reference order, not bit for bit; norms_separate keeps its order). "
                "tune_us = [library, chosen] per call"}
    del g, st, wts, xbuf, mm
    torch.cuda.empty_cache()

    # Codec window transformer (beside configs C1-C5): the same kernels on a 128-position
    # ring with caches that are views into a per-row byte arena (fast_engine.py:337-341, 368-387, 470-477),
    # 192 rows with a full window (lens 128, positions past the wrap). The codec's own head shape needs the
    # checkpoint (absent offline), so the slow stack's 14 / 2 x 64 stands in.
    b, S, layers = 192, 128, 4
    st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=b, cache_rows=b, cache_len=S, max_pos=4096, dev=dev,
                      nsplit_max=1, ring=S)
    per = NKV * S * HD
    arena = torch.zeros(b, layers * 2 * (per + 8), dtype=torch.bfloat16, device=dev)
    for i in range(layers):
        o = i * 2 * (per + 8)
        st.kc[i] = arena[:, o:o + per].view(b, NKV, S, HD)
        st.vc[i] = arena[:, o + per + 8:o + 2 * per + 8].view(b, NKV, S, HD)
        st.kc[i].normal_(generator=gen)
        st.vc[i].normal_(generator=gen)
    pos = torch.full((b,), 1000, dtype=torch.int32, device=dev)
    lens_d = torch.full((b,), S, dtype=torch.int32, device=dev)
    slot = torch.arange(b, dtype=torch.int32, device=dev)
    qkv = [randn(b, W) for _ in range(layers)]
    bias = [randn(W, std=0.02) for _ in range(layers)]
    q = torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(b, NQ, HD, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    g = capture(torch, lambda: st.forward(qkv, bias, pos, slot, lens_d, nsplit=1, rowmap=False, q=q, outs=outs,
                                          fuse=True))
    us = time_median(torch, g, steps, 10) * 1e3 / layers
    nbytes = ref_counts.decode_bytes([S] * b, NQ, NKV, HD)
    res["codec_window"] = {"us_per_layer": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1), "rows": b,
                           "kv_len": S, "ring": S, "schedule": list(st.attn.schedule(b, S, fused=True)),
                           "note": "fused store + decode on the 128-position ring, arena-strided caches; "
                                   "latency bound (~13 MB per layer)"}
    del g, st, qkv, outs, arena
    torch.cuda.empty_cache()

    # Streaming codec decoder (beside configs C1-C5): one codec frame (4 decoder input rows after the x4
    # upsample) for 192 rows through the channels-last conv stack, one graph. The checkpoint's decoder is absent
    # offline: a synthetic DAC-style decoder (1024 -> 1536 channels, strides 8, 8, 4, 2, kernel 7, dilations
    # 1, 3, 9) stands in. FLOPs count each conv's multiply-adds (2 B T_out Cout taps Cin).
    voc = import_module(a8.__name__ + ".vocoder")
    b, T = 192, 4
    wts = voc.decoder_weights(dev=dev, seed=21)
    dec = voc.CLDecoder(wts, b, dev, fused_ru=voc.FusedRU.DEFAULT_WIDTHS)
    xf = torch.randn(b, T, 1024, generator=gen, device=dev).to(torch.float16)
    g = capture(torch, lambda: dec(xf, b))
    us = time_median(torch, g, max(steps // 5, 5), 3) * 1e3
    flops, t, C = 2 * b * T * 1536 * 7 * 1024, T, 1536
    for _, _, _, s, units in wts["blocks"]:
        flops += 2 * b * t * s * (C // 2) * 2 * C
        t, C = t * s, C // 2
        flops += len(units) * 2 * b * t * C * C * 8
    flops += 2 * b * t * 1 * 7 * C
    del g
    # the same frame with every residual unit as its two convs (fused_ru=(): the reference's default path)
    dec2 = voc.CLDecoder(wts, b, dev, fused_ru=())
    g = capture(torch, lambda: dec2(xf, b))
    us_two = time_median(torch, g, max(steps // 5, 5), 3) * 1e3
    del g
    # the dominant launches: a residual unit at the 192-channel block (1024 output rows per row), as its k=7
    # conv alone (two-conv path) and as the whole fused unit
    c1, c2, fu = dec.blocks[2][1][0]
    xr = torch.randn(b, 1024, 192, generator=gen, device=dev).to(torch.float16)
    g = capture(torch, lambda: c1(xr, b))
    us_c = time_median(torch, g, steps, 10) * 1e3
    del g
    g = capture(torch, lambda: c2(c1(xr, b), b, res=xr))
    us_u2 = time_median(torch, g, steps, 10) * 1e3
    del g
    g = capture(torch, lambda: fu(xr, b))
    us_ru = time_median(torch, g, steps, 10) * 1e3
    fl_c = 2 * b * 1024 * 192 * 7 * 192
    fl_u = fl_c + 2 * b * 1024 * 192 * 192
    res["vocoder_frame"] = {"us_per_frame": round(us, 1), "TFLOP/s": round(flops / us / 1e6, 1),
                            "frac_fp16_mfma": round(flops / us / 1e6 / 2500.0, 4), "rows": b, "flops": flops,
                            "us_per_frame_two_conv_units": round(us_two, 1),
                            "conv_k7_c192": {"us": round(us_c, 1), "TFLOP/s": round(fl_c / us_c / 1e6, 1),
                                             "note": "snake_cat + conv_cl + state copy, M = 196608, N = 192, "
                                                     "K = 1344"},
                            "unit_c192": {"fused_us": round(us_ru, 1), "two_conv_us": round(us_u2, 1),
                                          "fused_TFLOP/s": round(fl_u / us_ru / 1e6, 1),
                                          "note": "one residual unit, 192 rows x 1024 positions x 192 channels: "
                                                  "snake_cat + ru_cl + state copy vs the k=7 and 1x1 convs"},
                            "note": "one frame of the streaming decoder; synthetic DAC-style weights; residual "
                                    "units of 96 / 192 channels fused (ru_cl, opted in: the reference's default "
                                    "and CLDecoder's are two convs, us_per_frame_two_conv_units; the fused unit "
                                    "keeps the first conv's output in fp32), the 384 / 768-channel ones two convs"}
    del g, dec, dec2, wts, xf, xr
    torch.cuda.empty_cache()

    # C4: 64 requests, n ~ U[40, 400], after a 300-position voice prefix; store + packed prefill per layer
    ns = torch.randint(40, 401, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    p0, nreq, layers = 300, 64, LAYERS
    R, S = sum(ns), 704
    st = a8.AttnStack(layers, NQ, NKV, HD, 10000.0, max_rows=8192, cache_rows=nreq + 1, cache_len=S, max_pos=S,
                      dev=dev)
    for i in range(layers):
        st.kc[i].normal_(generator=gen)
        st.vc[i].normal_(generator=gen)
    pos = torch.cat([p0 + torch.arange(n) for n in ns]).int().to(dev)
    slot = torch.cat([torch.full((n,), i) for i, n in enumerate(ns)]).int().to(dev)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    plan = a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev)
    qkv = [randn(R, W) for _ in range(layers)]
    bias = [randn(W, std=0.02) for _ in range(layers)]
    q = torch.empty(R, NQ, HD, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(R, NQ, HD, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    # the engine's path: k / v stored, q formed inside the prefill (fuse=True); beside it the two-step form
    # (q written by the store, then read by the prefill), which leaves the same bits
    g = capture(torch, lambda: st.forward(qkv, bias, pos, slot, None, plan=plan, q=q, outs=outs, fuse=True))
    us = time_median(torch, g, steps, 10) * 1e3 / layers
    del g
    g = capture(torch, lambda: st.forward(qkv, bias, pos, slot, None, plan=plan, q=q, outs=outs))
    us_unfused = time_median(torch, g, steps, 10) * 1e3 / layers
    del g

    def pf_only():
        for i in range(layers):
            a8.prefill_attention(q, st.kc[i], st.vc[i], plan, outs[i], NQ // NKV)

    def pf_qkv_only():
        for i in range(layers):
            a8.prefill_attention_qkv(qkv[i], bias[i], st.cos, st.sin, st.kc[i], st.vc[i], plan, outs[i], NQ // NKV)

    g = capture(torch, pf_qkv_only)
    us_pf_qkv = time_median(torch, g, steps, 10) * 1e3 / layers
    del g
    g = capture(torch, pf_only)
    us_pf = time_median(torch, g, steps, 10) * 1e3 / layers
    flops = ref_counts.prefill_flops(ns, [p0] * nreq, NQ, HD)
    # the admission step before it: the voices' prefix K/V into the 64 slots (4 voices x 16 slots, all layers;
    # fast_engine.py:1098-1103), one a8_prefix_copy per voice, against the reference's torch index-puts
    pk = [randn(layers, NKV, p0, HD) for _ in range(4)]
    pv = [randn(layers, NKV, p0, HD) for _ in range(4)]
    groups = [torch.arange(16 * j, 16 * j + 16, dtype=torch.int32, device=dev) for j in range(4)]

    def pcopy():
        for j in range(4):
            a8.prefix_copy(pk[j], pv[j], st.kc_all, st.vc_all, groups[j])

    def pcopy_torch():
        for j in range(4):
            idx = groups[j].long()
            st.kc_all[:, idx, :, :p0] = pk[j].unsqueeze(1)
            st.vc_all[:, idx, :, :p0] = pv[j].unsqueeze(1)

    g = capture(torch, pcopy)
    us_pc = time_median(torch, g, steps, 10) * 1e3
    del g
    g = capture(torch, pcopy_torch)
    us_pc_torch = time_median(torch, g, steps, 10) * 1e3
    pc_bytes = 2 * layers * NKV * p0 * HD * 2 * (nreq + 4)  # K+V written into 64 slots + the 4 prefixes read
    res["C4"] = {"us_per_layer": round(us, 3), "unfused_us_per_layer": round(us_unfused, 3),
                 "prefill_us_per_layer": round(us_pf, 3), "prefill_qkv_us_per_layer": round(us_pf_qkv, 3),
                 "prefix_copy": {"us": round(us_pc, 3), "GB/s": round(pc_bytes / us_pc / 1e3, 1),
                                 "frac_hbm": round(pc_bytes / us_pc / 1e3 / HBM_PEAK_GBS, 4), "bytes": pc_bytes,
                                 "torch_index_put_us": round(us_pc_torch, 3),
                                 "note": "4 voices x 16 slots x 24 layers x 300 positions, K and V"},
                 "prefill_TFLOP/s": round(flops / us_pf / 1e6, 1),
                 "frac_mfma_bf16": round(flops / us_pf / 1e6 / MFMA_BF16_TFLOPS, 4), "flops_per_layer": flops,
                 "rows": R, "blocks": plan.nblk,
                 "note": "us_per_layer: the k / v store + the prefill forming q from the qkv rows (fuse=True); "
                         "unfused: the store writing q too, then the prefill reading it (same bits); prefill_*: the "
                         "launch alone over a stored q / over the qkv rows; the prefill's fp32 softmax VALU work "
                         "bounds it before MFMA does"}
    if cpu_budget > 0:  # the CPU oracle on layer 0: store, then the packed prefill (prefix already in the caches)
        kc_h, vc_h = st.kc[0].cpu(), st.vc[0].cpu()
        qkv_h, bias_h, pos_h, slot_h = qkv[0].cpu(), bias[0].cpu(), pos.cpu(), slot.cpu()
        cos_h, sin_h = ref_counts.rope_tables(10000.0, HD, S)
        pl = ref_counts.prefill_plan(r0s, ns, list(range(nreq)), [p0] * nreq)

        def cpu_prefill():
            qh = torch.empty(R, NQ, HD, dtype=torch.bfloat16)
            ref_counts.bias_rope_store(qkv_h, bias_h, cos_h, sin_h, pos_h, slot_h, qh, kc_h, vc_h, NQ, NKV, HD)
            oh = torch.empty(R, NQ, HD, dtype=torch.bfloat16)
            ref_counts.prefill_attention(qh, kc_h, vc_h, *pl, oh, NQ // NKV)

        res["C4"]["cpu_baseline"] = cpu_leg(cpu_prefill, flops, "GFLOP/s", cpu_budget,
                                            f"1 of {layers} layers (store + packed prefill, {R} rows, same inputs)")
    del g, st, qkv, outs
    torch.cuda.empty_cache()
    res["hd128"] = hd128_configs(a8, torch, dev, steps, gen)
    return res


def hd128_configs(a8, torch, dev, steps, gen):
    """head_dim 128 (the fast AR's head width comes from its checkpoint, fast_engine.py:608, and 128 is the
    other width the kernels serve): the C3 decode load, the C5 fast-AR passes and the C4 packed prefill at
    head_dim 128 with the slow stack's 14 / 2 heads, 8 layers per graph. At this width the store is its own
    launch (the fused store + decode kernels are head_dim 64) and every launch is k_attn_cols<128>. µs per
    layer (per pass-layer), GB/s or TFLOP/s and the roofline fraction."""
    from oracle import attn_ref as ref_counts  # byte / FLOP counts only
    hd, layers = 128, 8
    w128 = (NQ + 2 * NKV) * hd

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(torch.bfloat16)

    out = {}
    # decode: 192 rows x KV 2048 (C3's load), store + decode per layer and the decode launch alone
    b, S = 192, 2048
    st = a8.AttnStack(layers, NQ, NKV, hd, 10000.0, max_rows=16 * b, cache_rows=b + 1, cache_len=S, max_pos=S,
                      dev=dev)
    for i in range(layers):
        st.kc[i].normal_(generator=gen)
        st.vc[i].normal_(generator=gen)
    lens = torch.full((b,), S, dtype=torch.int32, device=dev)
    pos, slot = lens - 1, torch.arange(b, dtype=torch.int32, device=dev)
    qkv = [randn(b, w128) for _ in range(layers)]
    bias = [randn(w128, std=0.02) for _ in range(layers)]
    q = torch.empty(b, NQ, hd, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(b, NQ, hd, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    nsplit = a8.ref_nsplit(b, NKV)
    g = capture(torch, lambda: st.forward(qkv, bias, pos, slot, lens, nsplit=nsplit, rowmap=False, q=q, outs=outs,
                                          fuse=True))
    us = time_median(torch, g, steps, 10) * 1e3 / layers
    del g

    def dec_only():
        for i in range(layers):
            st.attn(q, st.kc[i], st.vc[i], lens, outs[i], nsplit)

    g = capture(torch, dec_only)
    us_d = time_median(torch, g, steps, 10) * 1e3 / layers
    del g
    nb = ref_counts.decode_bytes([S] * b, NQ, NKV, hd)
    nb_d = ref_counts.decode_bytes([S] * b, NQ, NKV, hd, with_store=False)
    out["decode_192x2048"] = {"us_per_layer": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                              "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4), "bytes_per_layer": nb,
                              "decode_us_per_layer": round(us_d, 3),
                              "decode_frac_hbm": round(nb_d / us_d / 1e3 / HBM_PEAK_GBS, 4),
                              "note": "store (k_bias_rope_store) + decode (k_attn_cols<128>, one workgroup per "
                                      "16 query columns)"}
    del st, qkv, outs
    torch.cuda.empty_cache()
    # fast-AR passes (C5's shape): 192 slots, cache 10, a 2-token pass then 8 one-token passes
    b, S, nl = 192, 10, 4
    st = a8.AttnStack(nl, NQ, NKV, hd, 10000.0, max_rows=4 * b, cache_rows=b, cache_len=S, max_pos=16, dev=dev,
                      nsplit_max=1)
    r = torch.arange(2 * b, dtype=torch.int32)
    passes = [((r % 2).to(dev), (r // 2).to(dev), (r % 2 + 1).to(dev), True, 2 * b)]
    for p in range(2, 10):
        passes.append((torch.full((b,), p, dtype=torch.int32, device=dev), torch.arange(b, dtype=torch.int32,
                       device=dev), torch.full((b,), p + 1, dtype=torch.int32, device=dev), False, b))
    qkvs = [[randn(nr, w128) for _ in range(nl)] for (_, _, _, _, nr) in passes]
    bias = [randn(w128, std=0.02) for _ in range(nl)]
    q = torch.empty(2 * b, NQ, hd, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(2 * b, NQ, hd, dtype=torch.bfloat16, device=dev) for _ in range(nl)]

    def c5():
        for (ps, sl, ln, rmap, nr), qk in zip(passes, qkvs):
            st.forward(qk, bias, ps, sl, ln, nsplit=1, rowmap=rmap, q=q[:nr], outs=[o[:nr] for o in outs],
                       fuse=not rmap)

    g = capture(torch, c5)
    us = time_median(torch, g, steps, 10) * 1e3 / (len(passes) * nl)
    del g, st, qkvs, outs
    torch.cuda.empty_cache()
    out["fast_ar_passes"] = {"us_per_pass_layer": round(us, 3), "passes": len(passes), "layers": nl, "rows": b,
                             "note": "C5's passes at head_dim 128: store + decode per pass-layer, latency bound"}
    # packed prefill at C4's shape
    import numpy as np
    ns = torch.randint(40, 401, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    p0, nreq = 300, 64
    R, S = sum(ns), 704
    st = a8.AttnStack(layers, NQ, NKV, hd, 10000.0, max_rows=8192, cache_rows=nreq + 1, cache_len=S, max_pos=S,
                      dev=dev)
    for i in range(layers):
        st.kc[i].normal_(generator=gen)
        st.vc[i].normal_(generator=gen)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    plan = a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev)
    q = randn(R, NQ, hd)
    outs = [torch.empty(R, NQ, hd, dtype=torch.bfloat16, device=dev) for _ in range(layers)]

    def pf_only():
        for i in range(layers):
            a8.prefill_attention(q, st.kc[i], st.vc[i], plan, outs[i], NQ // NKV)

    g = capture(torch, pf_only)
    us_pf = time_median(torch, g, steps, 10) * 1e3 / layers
    del g, st, outs
    torch.cuda.empty_cache()
    flops = ref_counts.prefill_flops(ns, [p0] * nreq, NQ, hd)
    out["prefill_c4"] = {"us_per_layer": round(us_pf, 3), "TFLOP/s": round(flops / us_pf / 1e6, 1),
                         "frac_mfma_bf16": round(flops / us_pf / 1e6 / MFMA_BF16_TFLOPS, 4), "flops_per_layer": flops,
                         "note": "C4's 64 requests after a 300-position prefix, packed prefill alone"}
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_c3_traffic.md")


def measured_traffic(cfg, launch):
    """HBM bytes per launch of the decode kernel, from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes over
    `bench.py --traffic-probe` summarised in profiles/decode_c3_traffic.md (counters cannot be read from
    inside a timed run); None when that summary is absent or was taken at another config or launch shape."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    fields = dict(m.groups() for m in re.finditer(r"^- (\w+): `?([^`\n]+)`?$", text, re.M))
    if fields.get("config") != cfg or fields.get("launch") != json.dumps(launch, sort_keys=True):
        return None
    return int(fields["traffic_bytes_per_launch"])


def traffic_probe(torch, st, w, nsplit_req):
    """Counter target for the traffic measurement: 4 launches of one layer of the tick (the bench's launch:
    store + decode) and a plain 256 MiB elementwise copy (read 256 MiB, write 256 MiB) that calibrates
    FETCH_SIZE / WRITE_SIZE to bytes. Run under rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE."""
    for _ in range(4):
        st.layer(0, w["qkv"][0], w["bias"][0], w["pos"], w["slot"], w["lens"], w["q"], w["outs"][0],
                 nsplit=nsplit_req, rowmap=False, fuse=True)
    x = torch.ones(64 << 20, dtype=torch.float32, device=w["q"].device)
    y = torch.empty_like(x)
    for _ in range(2):
        torch.add(x, 0.0, out=y)
    torch.cuda.synchronize()
    print("traffic probe: 4 tick-layer launches, 2 copies of 268435456 bytes", flush=True)


def vocoder_probe(a8, torch, dev):
    """Profile target for the vocoder convolutions: the synthetic DAC-style decoder (1024 -> 1536 channels,
    strides 8, 8, 4, 2) run eagerly for 5 frames of 4 input rows at 192 rows."""
    from importlib import import_module
    voc = import_module(a8.__name__ + ".vocoder")
    b = 192
    dec = voc.CLDecoder(voc.decoder_weights(dev=dev, seed=21), b, dev, fused_ru=voc.FusedRU.DEFAULT_WIDTHS)
    gen = torch.Generator(device=dev).manual_seed(5)
    xf = torch.randn(b, 4, 1024, generator=gen, device=dev).to(torch.float16)
    for _ in range(5):
        dec(xf, b)
    torch.cuda.synchronize()
    print("vocoder probe: 5 frames done", flush=True)


def slow_probe(a8, torch, dev, shapes=None):
    """Profile target for the slow-AR step's projections: the 24-layer step at 192 rows x KV 2048 (synthetic
    weights, as the slow_ar_step leg) with GemmDispatch tuned first and the norms inside the projections, then 3 steps
    replayed from a graph."""
    from importlib import import_module
    ss = import_module(a8.__name__ + ".slow_stack")
    b, S, layers, hidden, inter = 192, 2048, LAYERS, 896, 4864
    wts, norm = ss.random_weights(layers, hidden, NQ, NKV, HD, inter, dev, seed=11)
    st = a8.SlowStack(wts, norm, NQ, NKV, HD, 1e-6, 10000.0, max_rows=max(16 * b, 8192), cache_rows=b + 1,
                      cache_len=S, max_pos=S, dev=dev)
    mm = a8.GemmDispatch()
    mm.tune([L[k] for L in wts for k in ("wqkv", "wo", "w13", "w2")], [b], gated=[L["w13"] for L in wts])
    for item in (shapes.split(",") if shapes else []):
        nk, sp, mb = item.split(":")
        N, K = (int(v) for v in nk.split("x"))
        mm.small_best[(b, N, K)] = (int(sp), int(mb))
        if (b, N, K) in mm.gated_best:
            mm.gated_best[(b, N, K)] = (1, int(mb))
    st.mm = mm
    st.fuse_norm = True
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(b, hidden, generator=gen, device=dev).to(torch.bfloat16)
    lens_d = torch.full((b,), S, dtype=torch.int32, device=dev)
    pos, slot = lens_d - 1, torch.arange(b, dtype=torch.int32, device=dev)
    g = capture(torch, lambda: st.forward(x, pos, slot, lens_d, rowmap=False, fuse=True))
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    print("slow probe: gemm_small shapes", {f"{N}x{K}": c for (M, N, K), c in mm.small_best.items()},
          "gated", {f"{N}x{K}": c for (M, N, K), c in mm.gated_best.items()}, flush=True)


def prefill_probe(a8, torch, dev):
    """Counter target for the prefill: the C4 workload (64 requests, n ~ U[40, 400] after a 300-position
    prefix, 13,745 packed rows) launched 3 times over a stored q, then 3 times forming q from qkv rows, then 3
    times at head_dim 128. Run under rocprofv3 --pmc with one counter group a pass."""
    import numpy as np
    g = torch.Generator(device=dev).manual_seed(7)
    ns = torch.randint(40, 401, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    p0, S, nreq = 300, 704, 64
    R = sum(ns)
    kc = torch.randn(nreq + 1, NKV, S, HD, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(nreq + 1, NKV, S, HD, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(R, NQ, HD, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    r0s = [int(x) for x in np.cumsum([0] + ns[:-1])]
    plan = a8.PrefillPlan(r0s, ns, list(range(nreq)), [p0] * nreq, dev)
    for _ in range(3):
        a8.prefill_attention(q, kc, vc, plan, out, NQ // NKV)
    # then the launch forming q from qkv rows (the k / v columns unused here), 3 times
    W = (NQ + 2 * NKV) * HD
    qkv = torch.randn(R, W, generator=g, device=dev).to(torch.bfloat16)
    bias = (0.02 * torch.randn(W, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = a8.rope_tables(10000.0, HD, S, dev)
    for _ in range(3):
        a8.prefill_attention_qkv(qkv, bias, cos, sin, kc, vc, plan, out, NQ // NKV)
    # and the same plan at head_dim 128 (k_prefill128), 3 times
    kc2 = torch.randn(nreq + 1, NKV, S, 128, generator=g, device=dev).to(torch.bfloat16)
    vc2 = torch.randn(nreq + 1, NKV, S, 128, generator=g, device=dev).to(torch.bfloat16)
    q2 = torch.randn(R, NQ, 128, generator=g, device=dev).to(torch.bfloat16)
    out2 = torch.empty_like(q2)
    for _ in range(3):
        a8.prefill_attention(q2, kc2, vc2, plan, out2, NQ // NKV)
    torch.cuda.synchronize()
    print(f"prefill probe: 3 + 3 + 3 launches (q stored / q from qkv / head_dim 128), {R} rows, {plan.nblk} blocks",
          flush=True)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus}). Each GPU "
              "serves its own slots with no exchange, so N GPUs give N times the one-GPU value.", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__
    __graft_entry__.ensure_built()
    a8 = __graft_entry__.load_package()
    from oracle import attn_ref as ref_counts  # byte counts only (the timed GPU path never touches it)

    dev = torch.device("cuda:0")
    if args.prefill_probe:
        prefill_probe(a8, torch, dev)
        return
    if args.vocoder_probe:
        vocoder_probe(a8, torch, dev)
        return
    if args.slow_probe:
        slow_probe(a8, torch, dev, args.gemm_shapes)
        return
    props = torch.cuda.get_device_properties(dev)
    w = build_workload(a8, torch, args.config, dev)
    st, b = w["st"], w["b"]
    if args.shape:
        st.attn.force_shape = tuple(int(x) for x in args.shape.split(","))
    if args.stream_shape:
        st.attn.force_stream = tuple(int(x) for x in args.stream_shape.split(","))
    nsplit_req = a8.ref_nsplit(b, NKV)
    kind, shape = st.attn.schedule(b, w["S"], nsplit_req, fused=True)
    fused = kind == "stream"
    if kind == "stream":
        nw, tpw, grid = shape
        chunks = -(-w["S"] // (nw * tpw * 64))
        rows = chunks == 1 and nw == 4  # whole rows per workgroup: the whole-row kernel
        launch = {"kernel": ("k_decode_rows" if rows else "k_decode_stream") + (" (store fused)" if fused else "") +
                  (" + k_decode_stream_combine" if chunks > 1 else ""), "waves": nw,
                  "tiles_per_wave": tpw, "grid": grid, "chunk_keys": nw * tpw * 64, "chunks_per_row": chunks}
    else:
        ns, nw = shape
        launch = {"kernel": "k_bias_rope_store + k_decode_split" + ("" if ns == 1 else " + k_decode_combine"),
                  "nsplit": ns, "waves": nw}
    if args.traffic_probe:
        traffic_probe(torch, st, w, nsplit_req)
        return

    def tick():
        # the engine's slow tick (fast_engine.py:752-753: slot = arange, rowmap off); one slot per row, so the
        # store and the decode run as one launch where the schedule allows
        st.forward(w["qkv"], w["bias"], w["pos"], w["slot"], w["lens"], nsplit=nsplit_req, rowmap=False, q=w["q"],
                   outs=w["outs"], fuse=True)

    def decode_only():
        for i in range(LAYERS):
            st.attn(w["q"], st.kc[i], st.vc[i], w["lens"], w["outs"][i], nsplit=nsplit_req)

    def store_only():
        for i in range(LAYERS):
            a8.bias_rope_store(w["qkv"][i], w["bias"][i], st.cos, st.sin, w["pos"], w["slot"], w["q"], st.kc[i],
                               st.vc[i], NQ, NKV, HD)

    g_tick = capture(torch, tick)
    ms = time_median(torch, g_tick, args.steps, args.warmup)
    g_dec = capture(torch, decode_only)
    ms_dec = time_median(torch, g_dec, args.steps, args.warmup)
    g_sto = capture(torch, store_only)
    ms_sto = time_median(torch, g_sto, args.steps, args.warmup)
    del g_tick, g_dec, g_sto

    traffic = measured_traffic(args.config, launch)
    lens = w["lens_h"].tolist()
    layer_bytes = ref_counts.decode_bytes(lens, NQ, NKV, HD)                  # store + decode, algorithmic
    dec_bytes = ref_counts.decode_bytes(lens, NQ, NKV, HD, with_store=False)  # K+V read + q in + out
    us_layer = ms * 1e3 / LAYERS
    gbs = layer_bytes * LAYERS / (ms * 1e-3) / 1e9
    dec_us = ms_dec * 1e3 / LAYERS
    dec_gbs = dec_bytes / (dec_us * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.config}: {b} slots x KV {max(lens)}" + (" (U[128,2048])" if args.config == "C2"
                   else "") + f", GQA {NQ}/{NKV} hd {HD}, {LAYERS} layers x (bias_rope_store + split-K decode) "
                   "as one HIP graph tick" + (", store fused into the decode launch" if kind == "stream" else ""), "slots": b, "kv_len": max(lens), "cache_len": w["S"], "layers": LAYERS,
                   "decode_launch": launch},
        "us_per_layer": round(us_layer, 3),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        # the tick's one launch per layer (the fused store + decode at C3): algorithmic store + decode bytes
        # over its per-launch time inside the timed tick
        "roofline": {"bound": "hbm", "kernel": launch["kernel"],
                     "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": layer_bytes, "us_per_launch": round(us_layer, 3)},
        # the same tick as the reference's two launches per layer, and the decode launch alone
        "unfused": {"decode_us_per_layer": round(dec_us, 3), "decode_gbs": round(dec_gbs, 2),
                    "decode_frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                    "store_us_per_layer": round(ms_sto * 1e3 / LAYERS, 3)},
        "timing": f"median of 5 runs of {args.steps} graph replays (HIP events on the launching stream)",
        "device": {"name": props.name, "arch": getattr(props, "gcnArchName", ""), "cus": props.multi_processor_count},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    if not args.no_configs:
        buckets = bucket_sweep(a8, torch, w, args.steps)
        del st, w
        torch.cuda.empty_cache()
        line["per_config"] = per_config(a8, torch, dev, args.steps, 0.0 if args.no_cpu_baseline else 4.0)
        line["per_config"]["buckets_kv2048"] = buckets
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
