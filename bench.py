#!/usr/bin/env python3
"""Benchmark: aggregate decode tokens/s of the resident continuous decode step on one
MI355X, with the HBM roofline of the dominant kernel and the CPU oracle timed beside it.

Default workload (the north-star target): Llama-3-8B-shaped
decoder, Q4 block-32 weights, 128 continuous decode lanes with churn -- Poisson(4)
arrivals per step, prompts U[128,4096], outputs U[32,512] -- admitted onto a fixed fp16
page pool sized to 80% of free HBM.  Admitted prompts get synthetic fp16 K/V in their
reserved pages (standing in for a restored prefix).  The host control plane plans every
step up front; the timed region replays the device-resident schedule (fills, primes,
descriptor copies, one step graph per step) and is bracketed by a device sync.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pretrained-rstr_amd"))

from rstr import configs, hip, workload  # noqa: E402

METRIC = "aggregate decode tokens/sec at N lanes; % of HBM roofline (GB/s) on 1 MI355X"
HBM_PEAK_GBS = 8000.0

# attention split per workload (the split fixes the canonical reduction order, so it is a
# decoder parameter): the fastest of 16..1024 measured on MI355X for each workload
SPLITS = {"config5": 256, "config5_1lane": 64, "config3": 640, "config2": 32, "config4": 256, "prefill5": 256,
          "config1": 128,
          "chunk5": 256}

WORKLOADS = {
    # name: (model, lanes, page_size, maxpos, prompt range, output range, arrivals/step, seed)
    "config5": ("llama3_8b", 128, 16, 4096 + 512, (128, 4096), (32, 512), 4.0, 5),
    # the same model and request mix served by one lane (the weight-streaming regime)
    "config5_1lane": ("llama3_8b", 1, 16, 4096 + 512, (128, 4096), (32, 512), 4.0, 5),
    "config2": ("gemma3_270m", 16, 16, 2048 + 256 + 1, (64, 2048), (256, 256), 0.0, 1),
    # config 3: contexts log-uniform [256, 8192], lanes 0-31 fork one 1024-token prefix
    # (prompt/output None selects the shared-prefix planner)
    "config3": ("qwen3_06b", 64, 16, 8192 + 512, None, None, 0.0, 2),
}


# workloads whose route pages are a seeded random permutation of the physical pool
# ("Page tables are a random permutation of the physical page
# pool", permutation seed 1): the pool's own ids map through workload.PermutedPages
PAGE_PERM_SEEDS = {"config2": 1}

# isolated attention workloads: (model shape, lanes, seed)
ATTN_WORKLOADS = {"config4": ("llama3_8b", 128, 4)}


def attention_workload(args) -> dict:
    """Config 4: one layer's routed paged attention alone.  128 lanes of a
    Llama-3-8B-shaped layer (32/8 heads, hd 128), contexts lognormal(7, 1.2)
    clipped to [16, 32768] (seed 4), page ids permuted, and the first quarter of
    every lane's full pages drawn from one shared run of pages (a common prefix),
    so 25% of full pages are shared across lanes.  Reports logical and unique KV
    GB/s of the split kernel (merge timed beside it)."""
    sess = hip.Session(0)
    try:
        return _attention_workload(args, sess)
    finally:
        sess.close()  # also closes the model, pool and decoders on an error


def _attention_workload(args, sess) -> dict:
    name, B, seed = ATTN_WORKLOADS[args.workload]
    cfg = dict(configs.MODELS[name], n_layers=1)
    ps, n_kv, hd, n_q = 16, cfg["n_kv"], cfg["head_dim"], cfg["n_q"]
    lengths, pt, physical, shared_n, rng = workload.shared_prefix_routes(B, seed, page_size=ps)
    row_bytes = n_kv * hd * 2 * 2  # fp16 K + V of one token
    logical = int(lengths.sum()) * row_bytes
    unique_tokens = int(shared_n.max()) * ps + int((lengths - shared_n * ps).sum())
    unique = unique_tokens * row_bytes
    model = hip.Model(sess, cfg, seed=1)
    pool = hip.Pool(model, ps, physical)
    pool.fill_synthetic(np.arange(physical, dtype=np.int32), seed)
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    pool.attention_bench(0, q, pt, lengths, split=args.split, iters=max(1, args.warmup))
    split_ms, merge_ms = pool.attention_bench(0, q, pt, lengths, split=args.split, iters=args.steps)
    log(f"config4: {B} lanes, mean ctx {lengths.mean():.0f}, max {lengths.max()}, {physical} pages; "
        f"logical {logical / 1e9:.3f} GB, unique {unique / 1e9:.3f} GB per launch; "
        f"split {split_ms * 1e3:.1f} us, merge {merge_ms * 1e3:.1f} us")
    gbs = logical / (split_ms * 1e-3) / 1e9
    ugbs = unique / (split_ms * 1e-3) / 1e9
    out = {
        "metric": "paged attention KV GB/s (logical bytes per split launch); % of HBM roofline on 1 MI355X",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(split_ms + merge_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 KV, fp32 accumulate",
        "data": "synthetic (seeded fp16 page templates, N(0,1) queries)",
        "config": {"workload": f"config4: isolated paged attention, {B} lanes, {n_q}/{n_kv} heads, hd {hd}, "
                               "ctx lognormal(7,1.2) clipped [16,32768], 25% of full pages shared",
                   "lanes": B, "page_size": ps, "physical_pages": physical, "attention_split": args.split,
                   "mean_ctx": round(float(lengths.mean()), 1), "parallelism": "1 GPU (replica)"},
        "roofline": {"bound": "hbm", "achieved": round(ugbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ugbs / HBM_PEAK_GBS, 4), "traffic": attn_traffic(args.workload),
                     "kernel": "k_attn_split (unique KV bytes per launch)", "bytes_per_launch": unique,
                     "avg_launch_ms": round(split_ms, 4)},
        "logical_bytes_per_launch": logical, "merge_ms": round(merge_ms, 4),
    }
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_attention_baseline(q, lengths, ps, n_kv, hd, cfg["attn_scale"], args.split,
                                                         args.cpu_seconds)
        except Exception as e:  # the baseline must not hide the GPU number
            out["cpu_baseline"] = {"error": repr(e)}
    pool.close()
    model.close()
    sess.close()
    return out


# the reference CPU path's own configuration:
# (model, weight bits, prompt tokens, greedy steps, prompt seed)
CPU_WORKLOADS = {"config1": ("gemma3_270m", 8, 32, 64, 0)}


def config1_workload(args) -> dict:
    """Config 1: Gemma-3-270M-shaped Q8 decoder, one lane, a 32-token prompt of
    uniform ids (seed 0) primed token by token, then 64 greedy steps -- the run
    BASELINE.json defines on the reference CPU path.  The HIP decoder runs it
    through one rstr_step_lanes call per step (host-timed, tok/s = 1000 / median
    decode-step ms as continuation/benchmark.clj:180-194 reports); the oracle
    runs the same prompt with f32 K/V (decoder.clj:304-310) on all host cores,
    reported beside the host's STREAM-triad bandwidth, since one token streams
    every packed weight from host DRAM."""
    sess = hip.Session(0)
    try:
        return _config1_workload(args, sess)
    finally:
        sess.close()  # also closes the model, pool and decoders on an error


def _config1_workload(args, sess) -> dict:
    name, bits, P, G, seed = CPU_WORKLOADS[args.workload]
    cfg = configs.with_bits(configs.MODELS[name], bits)
    ps, maxpos, split = 16, P + G, args.split
    pps = -(-maxpos // ps)
    prompt = [int(x) for x in np.random.default_rng(seed).integers(0, cfg["vocab"], P)]

    def desc(t):
        return dict(slots=[(t // ps) * ps + t % ps], row_offsets=[0, 1], positions=[t],
                    page_table=[list(range(pps))], lengths=[t + 1], start_positions=[0])

    def run(dec):
        """Prompt token t is the input at position t; the last prompt position's
        argmax is the first generated token, and every later input is the
        previous step's argmax (the tail's resident row).  Returns (generated
        tokens, per-step seconds of the G decode steps)."""
        out, times = [], []
        dec.prime_lanes([0], [prompt[0]])
        for t in range(P + G - 1):
            t0 = time.perf_counter()
            tok = int(dec.step_lanes(**desc(t))[0])
            dt = time.perf_counter() - t0
            if t + 1 < P:
                dec.prime_lanes([0], [prompt[t + 1]])
            else:
                out.append(tok)
                times.append(dt)
        return out, times

    model = hip.Model(sess, cfg, seed=1)
    pool = hip.Pool(model, ps, pps)
    dec = hip.Decoder(model, pool, 1, pps, maxpos, split)
    for _ in range(max(1, args.warmup)):
        run(dec)  # the same positions are rewritten: each run is the full config
    gpu_tokens, times = run(dec)
    weight_bytes = model.weight_bytes
    dec.close()
    pool.close()
    model.close()
    sess.close()
    med = float(np.median(times))
    kv_bytes = np.mean([2 * cfg["n_layers"] * (t + 1) * cfg["n_kv"] * cfg["head_dim"] * 2 for t in range(P - 1, P + G - 1)])
    step_bytes = weight_bytes + kv_bytes
    gbs = step_bytes / med / 1e9
    log(f"config1: {G} greedy steps, median {med * 1e3:.3f} ms/step (mean {np.mean(times) * 1e3:.3f}), "
        f"{step_bytes / 1e6:.1f} MB/step")
    out = {
        "metric": METRIC, "value": round(1.0 / med, 1), "unit": "tokens/s", "n_gpus": 1, "steps": G,
        "warmup": args.warmup, "ms_per_step": round(med * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q8/int8 block dots exact, fp32 accumulate, fp16 KV",
        "data": "synthetic (seeded random-init weights, uniform prompt ids seed 0)",
        "config": {"workload": f"config1: {name}-shaped Q8 decoder, 1 lane, {P}-token prompt primed token by token, "
                               f"{G} greedy steps (one rstr_step_lanes call per step, host-timed median)",
                   "lanes": 1, "page_size": ps, "attention_split": split, "parallelism": "1 GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole step (packed weights + visible K/V per host-timed step)",
                     "bytes_per_launch": int(step_bytes), "avg_launch_ms": round(med * 1e3, 4)},
        "generated_tokens_head": gpu_tokens[:8],
    }
    if not args.no_cpu_baseline:
        try:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle as O  # checker / CPU baseline only
            om = O.Model(cfg, seed=1)
            od = O.Decoder(om, 1, ps, pps, pps, maxpos, kv_f16=False, split=split)
            t0 = time.perf_counter()
            cpu_tokens, cpu_times = run(od)
            el = time.perf_counter() - t0
            od.close()
            om.close()
            cpu_med = float(np.median(cpu_times))
            triad = float(O.lib().orc_stream_triad(1 << 26, 5))
            cpu_gbs = step_bytes / cpu_med / 1e9
            agree = sum(int(a == b) for a, b in zip(gpu_tokens, cpu_tokens))
            out["cpu_baseline"] = {
                "value": round(1.0 / cpu_med, 2), "unit": "tokens/s", "cores": int(O.lib().orc_num_threads()),
                "kind": "port",
                "sample": f"the whole config: {P} prompt + {G} greedy steps ({el:.1f} s), median decode step; "
                          f"f32 K/V as the reference CPU path keeps them",
                "host_stream_triad_gbs": round(triad, 1), "achieved_gbs": round(cpu_gbs, 1),
                "frac_of_triad": round(cpu_gbs / triad, 3) if triad > 0 else None,
                "greedy_tokens_equal_to_gpu": f"{agree}/{G}"}
        except Exception as e:  # the baseline must not hide the GPU number
            out["cpu_baseline"] = {"error": repr(e)}
    return out


# bulk prefill workloads: (model, tile rows T, prompt tokens, seed)
PREFILL_WORKLOADS = {"prefill5": ("llama3_8b", 512, 4096, 6)}


def prefill_workload(args) -> dict:
    """Bulk paged prefill (prefill-range!, paged_decoder.clj:638-711): a step is one
    4096-token prompt of a Llama-3-8B-shaped Q4 model written into a fresh route of
    permuted pages, ``T`` rows per tile through ``rstr_prefill_range`` (layers only).
    Each tile's rows are causal lanes: projections run as one M = T MFMA tile per
    linear, attention reads the route's pages up to each row."""
    sess = hip.Session(0)
    try:
        return _prefill_workload(args, sess)
    finally:
        sess.close()  # also closes the model, pool and decoders on an error


def _prefill_workload(args, sess) -> dict:
    name, T, P, seed = PREFILL_WORKLOADS[args.workload]
    cfg = configs.MODELS[name]
    ps = 16
    pps = P // ps
    rng = np.random.default_rng(seed)
    model = hip.Model(sess, cfg, seed=1)
    physical = 4 * pps
    pool = hip.Pool(model, ps, physical)
    pf = hip.Prefill(model, pool, T, pps, P, args.split)
    prompts = [rng.integers(0, cfg["vocab"], P).astype(np.int32) for _ in range(4)]
    tables = [rng.permutation(physical)[:pps].astype(np.int32) for _ in range(4)]

    def prefill(i):
        toks, pt = prompts[i % 4], tables[i % 4]
        for t0 in range(0, P, T):
            pos = np.arange(t0, t0 + T, dtype=np.int32)
            slots = pt[pos // ps] * ps + pos % ps
            pf.prefill_range(toks[t0:t0 + T], slots, pos, pt, t0 + T, 0)

    for i in range(args.warmup):
        prefill(i)
    t0 = time.perf_counter()
    for i in range(args.steps):
        prefill(i)
    dt = time.perf_counter() - t0
    value = args.steps * P / dt
    d, qd, kvd = cfg["d_model"], cfg["n_q"] * cfg["head_dim"], cfg["n_kv"] * cfg["head_dim"]
    per_layer = (qd + 2 * kvd) * d + d * qd + 2 * cfg["d_ff"] * d + d * cfg["d_ff"]
    linear = 2 * per_layer * cfg["n_layers"] * P
    attn = 4 * cfg["n_q"] * cfg["head_dim"] * cfg["n_layers"] * (P * (P + 1) // 2)
    tflops = (linear + attn) / (dt / args.steps) / 1e12
    log(f"{args.workload}: {args.steps} prompts of {P} tokens in {P // T} tiles of {T}: "
        f"{1e3 * dt / args.steps:.1f} ms/prompt, {value:.0f} tok/s, {tflops:.1f} TFLOP/s algorithmic")
    out = {
        "metric": "bulk prefill tokens/sec on 1 MI355X", "value": round(value, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4/int8 block dots exact, fp32 accumulate, fp16 KV",
        "data": "synthetic (seeded random-init weights, uniform random prompt ids)",
        "config": {"workload": f"{args.workload}: {name}-shaped Q4 decoder, one {P}-token prompt per step, "
                               f"prefill tiles of {T} rows (host call per tile, synchronous)",
                   "prefill_T": T, "prompt": P, "page_size": ps, "attention_split": args.split,
                   "parallelism": "1 GPU (replica)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None,
                     "kernel": "whole prefill (linear + causal attention flops per prompt / prompt time)"},
    }
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(cfg, prefix=P // 2, budget_s=args.cpu_seconds)
        except Exception as e:  # the baseline must not hide the GPU number
            out["cpu_baseline"] = {"error": repr(e)}
    pf.close()
    pool.close()
    model.close()
    sess.close()
    return out


# durable chunk workloads: (model, chunk tokens, route pages, seed)
CHUNK_WORKLOADS = {"chunk5": ("llama3_8b", 4096, 320, 7)}


def chunk_workload(args) -> dict:
    """KV chunk export/restore (page_pool.clj:1111-1374): a 4096-token durable
    chunk of a Llama-3-8B-shaped fp16 pool (32 layers x K/V, 2 KiB rows: 512 MiB
    payload) starting 5 tokens into a route of permuted pages.  ``value`` is the
    export rate through the C ABI, payload bytes over the transfer's device time
    (page list copy + gather kernel + device-to-host DMA into pinned memory);
    the roofline is the gather kernel alone (HBM: the payload read from pages
    and written to staging)."""
    sess = hip.Session(0)
    try:
        return _chunk_workload(args, sess)
    finally:
        sess.close()  # also closes the model, pool and decoders on an error


def _chunk_workload(args, sess) -> dict:
    name, T, npages, seed = CHUNK_WORKLOADS[args.workload]
    cfg = configs.MODELS[name]
    ps = 16
    rng = np.random.default_rng(seed)
    model = hip.Model(sess, cfg, seed=1)
    physical = 4 * npages
    pool = hip.Pool(model, ps, physical)
    pool.fill_synthetic(np.arange(physical, dtype=np.int32), seed)
    pages = rng.permutation(physical)[:npages].astype(np.int32)
    start = 5
    payload_bytes = pool.chunk_elements(T) * 2
    ex = [None]

    def export():
        st = pool.export_submit(pages, start, T).complete()
        ex[0] = st["payload"]
        return st["device_ms"]

    for _ in range(max(1, args.warmup)):
        export()
    t0 = time.perf_counter()
    dev = [export() for _ in range(args.steps)]
    wall = (time.perf_counter() - t0) / args.steps
    exp_ms = float(np.median(dev))
    other = np.setdiff1d(np.arange(physical), pages)[:npages].astype(np.int32)
    rdev = [pool.restore_submit(other, start, T, ex[0]).complete()["device_ms"] for _ in range(max(2, args.steps // 2))]
    res_ms = float(np.median(rdev))
    iters = max(10, args.steps)
    g_ms = pool.chunk_bench(pages, start, T, 0, iters)
    s_ms = pool.chunk_bench(other, start, T, 1, iters)
    gbs = payload_bytes / (exp_ms * 1e-3) / 1e9
    kern_gbs = 2 * payload_bytes / (g_ms * 1e-3) / 1e9
    log(f"{args.workload}: {T}-token chunk, {payload_bytes / 2**20:.0f} MiB: export {exp_ms:.2f} ms device "
        f"({gbs:.1f} GB/s, wall {1e3 * wall:.2f} ms), restore {res_ms:.2f} ms "
        f"({payload_bytes / (res_ms * 1e-3) / 1e9:.1f} GB/s); gather kernel {1e3 * g_ms:.1f} us "
        f"({kern_gbs:.0f} GB/s HBM), scatter kernel {1e3 * s_ms:.1f} us")
    out = {
        "metric": "durable KV chunk export GB/s (payload bytes / device time) on 1 MI355X",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(exp_ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 KV rows", "data": "synthetic (seeded fp16 page templates)",
        "config": {"workload": f"{args.workload}: {name}-shaped fp16 pool, one {T}-token chunk starting 5 tokens into "
                               f"a route of {npages} permuted 16-token pages; export = page list + gather kernel + "
                               "DMA to pinned host memory",
                   "chunk_tokens": T, "payload_bytes": payload_bytes, "page_size": ps,
                   "parallelism": "1 GPU (replica)"},
        "restore": {"device_ms": round(res_ms, 3), "gbs": round(payload_bytes / (res_ms * 1e-3) / 1e9, 2)},
        "export_wall_ms": round(1e3 * wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_chunk_move<0> (gather; payload read from pages + written to staging)",
                     "bytes_per_launch": 2 * payload_bytes, "avg_launch_ms": round(g_ms, 4),
                     "scatter_avg_launch_ms": round(s_ms, 4)},
    }
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_chunk_baseline(cfg, T, args.cpu_seconds)
        except Exception as e:  # the baseline must not hide the GPU number
            out["cpu_baseline"] = {"error": repr(e)}
    pool.close()
    model.close()
    sess.close()
    return out


def cpu_chunk_baseline(cfg, T, budget_s) -> dict:
    """The oracle's chunk gather (numpy fancy indexing over host slabs) on a
    1/8 sample of the chunk's tokens, all layers."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import chunk_oracle as OC  # checker / CPU baseline only
    ps, n = 16, T // 8
    ept = cfg["n_kv"] * cfg["head_dim"]
    npg = -(-(n + 5) // ps)
    rng = np.random.default_rng(3)
    slabs = [rng.integers(0, 2**15, (4 * npg * ps, ept)).astype(np.uint16) for _ in range(2 * cfg["n_layers"])]
    pages = rng.permutation(4 * npg)[:npg]
    reps, t0 = 0, time.perf_counter()
    while True:
        out = OC.gather(slabs, pages, ps, 5, n)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(out.nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} of {T} tokens, all {2 * cfg['n_layers']} slab-layers, {reps} gathers"}


def cpu_attention_baseline(q, lengths, ps, n_kv, hd, scale, split, budget_s) -> dict:
    """The oracle's routed attention (paged_attention.clj:196-228 restated in C,
    OpenMP over lanes) on host fp16 pages: lanes of the same workload taken in
    order until the sample holds about 1/16 of the logical bytes, repeated for
    about ``budget_s`` seconds."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker / CPU baseline only
    total = int(lengths.sum())
    n = 1
    while n < len(lengths) and int(lengths[:n].sum()) < total // 16:
        n += 1
    sub = lengths[:n]
    npg = -(-sub // ps)
    pt = np.full((n, int(npg.max())), -1, np.int32)
    off = 0
    for b in range(n):
        pt[b, :npg[b]] = np.arange(off, off + npg[b])
        off += int(npg[b])
    rng = np.random.default_rng(4)
    kp = rng.standard_normal((off, ps, n_kv, hd)).astype(np.float16)
    vp = rng.standard_normal((off, ps, n_kv, hd)).astype(np.float16)
    reps, t0 = 0, time.perf_counter()
    while True:
        O.attention(q[:n], kp, vp, pt, sub, 0, scale, split)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = (time.perf_counter() - t0) / reps
    nbytes = int(sub.sum()) * n_kv * hd * 2 * 2
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": int(O.lib().orc_num_threads()),
            "kind": "port",
            "sample": f"{n} of {len(lengths)} lanes ({int(sub.sum())} of {total} tokens), {reps} launches"}


def attn_traffic(workload_name):
    """HBM bytes per k_attn_split launch from the committed rocprofv3 FETCH_SIZE +
    WRITE_SIZE runs of this workload (profiles/attn_split_<workload>_traffic.json), or None."""
    tfile = os.path.join(ROOT, "profiles", f"attn_split_{workload_name}_traffic.json")
    if os.path.exists(tfile):
        return json.load(open(tfile)).get("hbm_bytes_per_launch")
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(cfg: dict, prefix: int, budget_s: float) -> dict:
    """The reference CPU path restated in C (oracle): Q4 int8-MAC linears, f32 KV, one
    lane at a time (decoder.clj:443-458 generate-cached), greedy; timed on this host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker / CPU baseline only
    t0 = time.perf_counter()
    model = O.Model(cfg, seed=1)
    build_s = time.perf_counter() - t0
    ps = 16
    pps = -(-(prefix + 256) // ps)
    dec = O.Decoder(model, 1, ps, pps, pps, prefix + 256, kv_f16=False, split=256)
    for pg in range(-(-prefix // ps)):
        dec.fill_synthetic(pg, 7)
    dec.prime_lanes([0], [1])
    steps, t1 = 0, time.perf_counter()
    length = prefix
    while True:
        length += 1
        t = length - 1
        desc = dict(slots=[(t // ps) * ps + t % ps], row_offsets=[0, 1], positions=[t],
                    page_table=[list(range(pps))], lengths=[length], start_positions=[0])
        dec.step_lanes(**desc)
        steps += 1
        el = time.perf_counter() - t1
        if el > budget_s or length >= prefix + 255:
            break
    threads = int(O.lib().orc_num_threads())
    dec.close()
    model.close()
    return {"value": round(steps / el, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"1 lane, {prefix}-token synthetic prefix, {steps} greedy decode steps "
                      f"({el:.1f} s; oracle model build {build_s:.1f} s untimed)"}


def linear_params(cfg: dict) -> tuple[int, int]:
    """(layer linear parameters over all layers, head parameters)."""
    d, ff, qd, kvr = cfg["d_model"], cfg["d_ff"], cfg["n_q"] * cfg["head_dim"], cfg["n_kv"] * cfg["head_dim"]
    return cfg["n_layers"] * (qd * d + 2 * kvr * d + d * qd + 2 * ff * d + d * ff), cfg["vocab"] * d


def class_rates(cfg: dict, prof: dict, n_steps: int, prof_plan: list, weight_bytes: int) -> dict:
    """Per kernel class: ms per step and, where the class has an algorithmic byte
    or flop count, GB/s and TFLOP/s.  Projections: packed weights and scales once
    per step, 2 flops per weight per active lane; attention: the visible fp16 K+V
    (unique pages), 4 * n_q * head_dim flops per visible token and layer."""
    layer_p, head_p = linear_params(cfg)
    per_w = (16 + 2) / 32 if cfg["weight_bits"] == 4 else (32 + 2) / 32
    head_bytes = int(head_p * per_w)
    rows = float(np.mean([st["active"] for st in prof_plan]))
    kv = float(np.mean([workload.step_bytes(cfg, st, 0).get("kv_unique", workload.step_bytes(cfg, st, 0)["kv"])
                        for st in prof_plan]))
    vis = float(np.mean([sum(workload.step_bytes(cfg, st, 0)["kv_per_layer"]) for st in prof_plan])) / (
        cfg["n_kv"] * cfg["head_dim"] * 4)
    work = {"qgemm": (weight_bytes - head_bytes, 2.0 * layer_p * rows),
            "head": (head_bytes, 2.0 * head_p * rows),
            "attn_split": (kv, 4.0 * cfg["n_q"] * cfg["head_dim"] * vis)}
    out = {}
    for k, (ms_tot, n) in prof.items():
        ms = ms_tot / n_steps
        e = {"ms_per_step": round(ms, 4), "launches_per_step": round(n / n_steps, 2)}
        if k in work and ms > 0:
            b, f = work[k]
            e["GB/s"] = round(b / (ms * 1e-3) / 1e9, 1)
            e["TFLOP/s"] = round(f / (ms * 1e-3) / 1e12, 2)
            e["bytes_per_step"] = int(b)
        out[k] = e
    return out


def live_loop(args, cfg, lanes, ps, physical, maxpos, prompt, output, arrivals, seed, dec, pool) -> dict:
    """The serving loop in the sense of continuation/benchmark.clj:180-194: every
    step is planned by the host control plane and run through one
    rstr_step_lanes call (descriptor upload, step graph, token download), timed
    per step from the host.  Reported beside the device-resident replay, with the
    host bookkeeping and the boundary call separated."""
    dev = workload.LiveDevice(dec, pool)
    planner = workload.ChurnPlanner(cfg, lanes, ps, physical, maxpos, seed=seed + 1000, arrival_mean=arrivals,
                                    prompt=prompt, output=output, device=dev,
                                    page_perm_seed=PAGE_PERM_SEEDS.get(args.workload))
    for _ in range(2):  # admissions of the steady-state start, first graph replays
        planner.plan_step()
    dev.step_seconds = dev.other_seconds = 0.0
    dev.phase_ms.clear()
    host0 = planner.host_seconds
    times = []
    for _ in range(args.live_steps):
        t0 = time.perf_counter()
        planner.plan_step()
        times.append(time.perf_counter() - t0)
    n = len(times)
    total = sum(times)
    step_s, other_s = dev.step_seconds, dev.other_seconds
    phases = {k: round(v / n, 4) for k, v in dev.phase_ms.items()}
    # idle probe: the last live step's descriptors again, back to back and with
    # the host pausing as long as the planner did between calls; the device time
    # of the same step graph tells the GPU's own ramp after idling apart from
    # the library's host work
    pause = max(0.0, (planner.host_seconds - host0 - step_s - other_s) / n)
    probe = {}
    for label, gap in (("back_to_back", 0.0), ("after_host_pause", pause)):
        dev_ms = []
        for _ in range(8):
            if gap:
                time.sleep(gap)
            dec.step_lanes(**dev._desc)
            dev_ms.append(dec.step_timing()["device_step"])
        probe[label] = round(float(np.median(dev_ms)), 4)
    probe["pause_ms"] = round(1e3 * pause, 3)
    piped = live_loop_pipelined(args, cfg, lanes, ps, physical, maxpos, prompt, output, arrivals, seed, dec, pool)
    return {"steps": n, "ms_per_step_median": round(1e3 * float(np.median(times)), 3),
            "ms_per_step_mean": round(1e3 * total / n, 3),
            "tokens_per_s_median": round(lanes / float(np.median(times)), 1) if lanes else None,
            "rstr_step_lanes_ms": round(1e3 * step_s / n, 3),
            "fills_copies_primes_ms": round(1e3 * other_s / n, 3),
            "host_bookkeeping_ms": round(1e3 * ((planner.host_seconds - host0) - step_s - other_s) / n, 3),
            # inside rstr_step_lanes (rstr_decoder_step_timing), mean ms per call
            "rstr_step_lanes_phases_ms": phases,
            # the same step's device time (ms, median of 8) back to back and after a host pause
            "idle_probe_device_step_ms": probe,
            "pipelined": piped}


def live_loop_pipelined(args, cfg, lanes, ps, physical, maxpos, prompt, output, arrivals, seed, dec, pool) -> dict:
    """The same serving loop with the host control plane one step ahead
    (workload.PipelinedLive): step n is submitted (rstr_step_lanes_submit), step
    n+1 is planned while the device runs it, applied and submitted before step
    n's tokens are collected, so the device receives the sequential loop's calls
    in the same order and the per-step time is the longer of the two instead of
    their sum.  Timed as the interval between consecutive collected steps."""
    planner = workload.ChurnPlanner(cfg, lanes, ps, physical, maxpos, seed=seed + 1000, arrival_mean=arrivals,
                                    prompt=prompt, output=output, page_perm_seed=PAGE_PERM_SEEDS.get(args.workload))
    loop = workload.PipelinedLive(planner, dec, pool)
    loop.start()
    for _ in range(2):  # admissions of the steady-state start, first graph replays
        loop.step()
    loop.plan_seconds = 0.0
    times = []
    t_prev = time.perf_counter()
    for _ in range(args.live_steps):
        loop.step()
        t = time.perf_counter()
        times.append(t - t_prev)
        t_prev = t
    loop.finish()
    n = len(times)
    return {"steps": n, "ms_per_step_median": round(1e3 * float(np.median(times)), 3),
            "ms_per_step_mean": round(1e3 * sum(times) / n, 3),
            "tokens_per_s_median": round(lanes / float(np.median(times)), 1) if lanes else None,
            "host_planning_ms": round(1e3 * loop.plan_seconds / n, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="config5", choices=sorted(WORKLOADS) + sorted(ATTN_WORKLOADS) + sorted(PREFILL_WORKLOADS)
                    + sorted(CHUNK_WORKLOADS) + sorted(CPU_WORKLOADS))
    ap.add_argument("--profile-steps", type=int, default=4)
    ap.add_argument("--pool-fraction", type=float, default=0.8)
    ap.add_argument("--split", type=int, default=None, help="attention split (default: per workload)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--live-steps", type=int, default=20, help="steps of the live serving loop (0: skip)")
    ap.add_argument("--no-extra", action="store_true",
                    help="config5 only: skip the config5_1lane, config2, config3, config1, config4 and prefill5 "
                         "sub-runs of the default line")
    args = ap.parse_args()
    if args.split is None:
        args.split = SPLITS[args.workload]
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (the decode step "
                                   "shards as independent per-GPU replicas with their own lanes and "
                                   "page pools, so one GPU's throughput is the per-replica figure)"}))
        sys.exit(2)

    if args.workload in ATTN_WORKLOADS:
        print(json.dumps(attention_workload(args)), flush=True)
        return
    if args.workload in PREFILL_WORKLOADS:
        print(json.dumps(prefill_workload(args)), flush=True)
        return
    if args.workload in CHUNK_WORKLOADS:
        print(json.dumps(chunk_workload(args)), flush=True)
        return
    if args.workload in CPU_WORKLOADS:
        print(json.dumps(config1_workload(args)), flush=True)
        return
    out = decode_workload(args)
    if args.workload == "config5" and not args.no_extra:
        # the other BASELINE configurations, measured in the same run (the driver
        # records one line); a sub-run that fails records its error and leaves the
        # config5 measurement intact
        out["other_workloads"] = {}

        def sub_run(name, fn, keys, **over):
            sub = argparse.Namespace(**vars(args))
            sub.workload, sub.split = name, SPLITS[name]
            for k, v in over.items():
                setattr(sub, k, v)
            try:
                r = fn(sub)
            except Exception as e:  # keep the headline line
                log(f"{name} sub-run failed: {e!r}")
                out["other_workloads"][name] = {"error": repr(e)}
                return
            if name == "config5_1lane" and "cpu_baseline" in out:
                # the oracle's one-lane Llama-3-8B decode is this workload's CPU baseline too
                r["cpu_baseline"] = dict(out["cpu_baseline"], sample="the config5 line's: "
                                         + out["cpu_baseline"].get("sample", ""))
            out["other_workloads"][name] = {k: r[k] for k in keys if k in r}

        decode_keys = ("value", "unit", "ms_per_step", "steps", "warmup", "config", "roofline", "step_roofline",
                       "kernel_ms_per_step", "kernel_classes", "live_loop", "cpu_baseline")
        for extra, steps in (("config5_1lane", 100), ("config2", 200), ("config3", 40)):
            sub_run(extra, decode_workload, decode_keys, steps=steps, warmup=10,
                    live_steps=min(args.live_steps, 10),
                    no_cpu_baseline=args.no_cpu_baseline or extra == "config5_1lane",
                    cpu_seconds=min(args.cpu_seconds, 6.0 if extra == "config2" else 4.0))
        sub_run("config1", config1_workload,
                ("value", "unit", "ms_per_step", "steps", "config", "roofline", "cpu_baseline"), warmup=1)
        sub_run("config4", attention_workload,
                ("metric", "value", "unit", "ms_per_step", "config", "roofline", "merge_ms", "cpu_baseline"),
                steps=20, warmup=3, cpu_seconds=min(args.cpu_seconds, 4.0))
        # the bulk prefill tile beside the step (chunk5 keeps its own line: its host-link
        # rate after the runs above reads ~30 GB/s against ~56 GB/s in a fresh process)
        sub_run("prefill5", prefill_workload,
                ("metric", "value", "unit", "ms_per_step", "config", "roofline", "cpu_baseline"),
                steps=2, warmup=1, cpu_seconds=min(args.cpu_seconds, 4.0))
    print(json.dumps(out), flush=True)


def decode_workload(args) -> dict:
    """One continuous-decode workload of WORKLOADS: plan on the host, replay the
    device-resident schedule in the timed region, profile, live loop, CPU baseline."""
    sess = hip.Session(0)
    try:
        return _decode_workload(args, sess)
    finally:
        sess.close()  # also closes the model, pool and decoders on an error


def _decode_workload(args, sess) -> dict:
    name, lanes, ps, maxpos, prompt, output, arrivals, seed = WORKLOADS[args.workload]
    cfg = configs.MODELS[name]
    pps = -(-maxpos // ps)
    t0 = time.perf_counter()
    model = hip.Model(sess, cfg, seed=1)
    log(f"model bound in {time.perf_counter() - t0:.1f}s, weights {model.weight_bytes / 1e9:.2f} GB")
    free, total = sess.memory()
    page_bytes = 2 * cfg["n_layers"] * ps * cfg["n_kv"] * cfg["head_dim"] * 2
    reserve = 8 << 30  # decoder scratch, templates, schedule
    physical = int(args.pool_fraction * (free - reserve) // page_bytes)
    t0 = time.perf_counter()
    pool = hip.Pool(model, ps, physical)
    log(f"page pool: {physical} pages x {page_bytes >> 20} MiB = {physical * page_bytes / 1e9:.1f} GB "
        f"({time.perf_counter() - t0:.1f}s)")
    dec = hip.Decoder(model, pool, lanes, pps, maxpos, args.split)

    # ---- plan the whole run on the host (control-plane mirror) -------------------------
    n_total = args.warmup + args.steps + args.profile_steps
    if prompt is None:
        planner = workload.SharedPrefixPlanner(cfg, lanes, ps, physical, maxpos, seed=seed)
    else:
        planner = workload.ChurnPlanner(cfg, lanes, ps, physical, maxpos, seed=seed, arrival_mean=arrivals,
                                        prompt=prompt, output=output,
                                        page_perm_seed=PAGE_PERM_SEEDS.get(args.workload))
    t0 = time.perf_counter()
    plan = [planner.plan_step() for _ in range(n_total)]
    plan_s = time.perf_counter() - t0
    host_ms_step = 1e3 * planner.host_seconds / n_total
    log(f"planned {n_total} steps in {plan_s:.1f}s ({host_ms_step:.2f} ms/step host bookkeeping), "
        f"retired {planner.retired}, rejected admissions {planner.rejected_admissions}")
    t0 = time.perf_counter()
    dec.schedule_upload(plan)
    log(f"schedule uploaded in {time.perf_counter() - t0:.1f}s")

    # ---- warmup, then the timed region ---------------------------------------------
    _, warm_ms = dec.schedule_run(0, args.warmup)
    log(f"warmup {args.warmup} steps: {warm_ms:.1f} ms (includes initial prefix fills)")
    toks, dev_ms = dec.schedule_run(args.warmup, args.steps)
    timed = plan[args.warmup:args.warmup + args.steps]
    tokens = sum(st["active"] for st in timed)
    ms_per_step = dev_ms / args.steps
    value = tokens / (dev_ms / 1e3)
    bytes_steps = [workload.step_bytes(cfg, st, model.weight_bytes) for st in timed]
    # unique physical KV rows (pages shared by lanes count once) where the step has a
    # page table without windows; logical rows otherwise
    step_bytes = float(np.mean([b.get("total_unique", b["total"]) for b in bytes_steps]))
    step_bytes_logical = float(np.mean([b["total"] for b in bytes_steps]))
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"timed {args.steps} steps: {dev_ms:.1f} ms, {ms_per_step:.3f} ms/step, {value:.0f} tok/s, "
        f"{step_bytes / 1e9:.2f} GB/step algorithmic -> {step_gbs:.0f} GB/s")

    # ---- per-kernel profile pass (eager, HIP events around each launch) -------------
    first = args.warmup + args.steps
    prof = dec.profile_steps(first, args.profile_steps)
    prof_plan = plan[first:first + args.profile_steps]
    def layer_kv(st):
        b = workload.step_bytes(cfg, st, 0)
        return b.get("kv_unique_per_layer", np.mean(b["kv_per_layer"]))
    attn_bytes = np.mean([layer_kv(st) for st in prof_plan])
    all_bytes = np.mean([layer_kv(st) for st in plan])
    log(f"attention algorithmic bytes per launch: {all_bytes:.0f} (all {len(plan)} steps), "
        f"{attn_bytes:.0f} (profiled steps)")
    attn_ms, attn_n = prof["attn_split"]
    attn_avg_ms = attn_ms / max(attn_n, 1)
    attn_gbs = attn_bytes / (attn_avg_ms * 1e-3) / 1e9
    qg_ms, qg_n = prof["qgemm"]
    log("profile (ms total / launches): " + ", ".join(f"{k} {v[0]:.2f}/{v[1]}" for k, v in prof.items()))

    classes = class_rates(cfg, prof, args.profile_steps, prof_plan, model.weight_bytes)
    dominant = max(("qgemm", "head", "attn_split"), key=lambda k: classes[k]["ms_per_step"])
    if dominant == "attn_split":
        traffic = attn_traffic(args.workload)
        roofline = {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "kernel": "k_attn_split (paged attention, per layer launch)",
                    "bytes_per_launch": int(attn_bytes), "avg_launch_ms": round(attn_avg_ms, 4)}
    else:
        c = classes[dominant]
        n_launch = prof[dominant][1] / args.profile_steps
        gbs = c["GB/s"]
        roofline = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": ("k_qgemm (dequantising projections, weight streaming)" if dominant == "qgemm"
                               else "k_qgemm (LM head)"),
                    "bytes_per_launch": int(c["bytes_per_step"] / n_launch),
                    "avg_launch_ms": round(c["ms_per_step"] / n_launch, 5)}
    live = None
    if args.live_steps > 0 and prompt is not None:
        live = live_loop(args, cfg, lanes, ps, physical, maxpos, prompt, output, arrivals, seed, dec, pool)
        log("live loop: " + json.dumps(live))

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4/int8 block dots exact, fp32 accumulate, fp16 KV",
        "data": "synthetic (seeded random-init weights, synthetic prefix K/V, "
                + ("Poisson churn)" if prompt is not None else "shared-prefix forks)"),
        "config": {"workload": (f"{args.workload}: {name}-shaped Q4 decoder, {lanes} continuous lanes, "
                                f"prompts U{list(prompt)}, outputs U{list(output)}, "
                                f"Poisson({arrivals}) arrivals/step"
                                + (f", route pages a seeded permutation of the physical pool (seed "
                                   f"{PAGE_PERM_SEEDS[args.workload]})" if args.workload in PAGE_PERM_SEEDS else
                                   ", pages lowest-free-first")) if prompt is not None else
                               (f"{args.workload}: {name}-shaped Q4 decoder, {lanes} decode lanes, contexts "
                                f"log-uniform[256, 8192], lanes 0-31 fork one 1024-token prefix "
                                f"(copy-on-write on the first divergent append); {planner.cow_pages} pages copied"),
                   "lanes": lanes, "page_size": ps, "physical_pages": physical,
                   "attention_split": args.split, "parallelism": "1 GPU (replica)"},
        "roofline": roofline,
        "step_roofline": {"bytes_per_step": int(step_bytes), "logical_bytes_per_step": int(step_bytes_logical),
                          "achieved_gbs": round(step_gbs, 1), "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "kernel_ms_per_step": {k: round(v[0] / args.profile_steps, 3) for k, v in prof.items()},
        "kernel_classes": classes,
        "host_bookkeeping_ms_per_step": round(host_ms_step, 3),
    }
    if live is not None:
        out["live_loop"] = live
    if not args.no_cpu_baseline:
        try:
            mean_ctx = int(np.mean(prompt)) if prompt is not None else int(np.mean(plan[0]["lengths"]))
            out["cpu_baseline"] = cpu_baseline(cfg, prefix=mean_ctx, budget_s=args.cpu_seconds)
        except Exception as e:  # the baseline must not hide the GPU number
            out["cpu_baseline"] = {"error": repr(e)}
    dec.close()
    pool.close()
    model.close()
    sess.close()
    return out


if __name__ == "__main__":
    main()
