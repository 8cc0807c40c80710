#!/usr/bin/env python3
"""Benchmark driver (one JSON line on stdout).

Default workload ``e2e`` (benchmark config 4, harness in ``bench_e2e.py``):
end-to-end batched beam search on a random-init Llama-3-8B-shaped decoder
(8 requests x beam 16, 1024-token prompts, 256 generated tokens); value =
beam-decode tokens/s = 128 candidate tokens per step / step time over
``--steps`` steps sampled evenly across the 256-step generation after
``--warmup`` untimed steps.  A step is one decode step of all 8 requests x 16
beams.  The flat strategy decodes the same prompts in the same process
(``config.flat``, ``config.vs_flat``).

Attention workloads (``--workload attn-c2|attn-ns|attn-c3|attn-c5|attn-c1``)
time one decode-attention layer at a benchmark shape over 32 distinct per-layer
KV caches (working set above the 256 MB Infinity Cache); value = algorithmic
HBM GB/s of the attention kernel.  ``--strategy flat`` runs the flat paged
strategy on the same pages.

Every line carries ``roofline`` (the attention kernel: algorithmic bytes per
launch / mean launch time from HIP events on the launch stream) and
``cpu_baseline`` (the CPU oracle on a bounded sample, rank 0, N=1 only).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=None, help="timed steps (decode steps / attention reps)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="e2e",
                    choices=["e2e", "attn-c1", "attn-c2", "attn-ns", "attn-c3", "attn-c5", "attn-e2e", "attn-prefill",
                             "topk", "topk-c1", "read-ns"])
    ap.add_argument("--strategy", default="cascade", choices=["cascade", "fasttree", "flat", "split", "tree", "auto"],
                    help="attention workloads: cascade or flat; e2e: also tree / auto (cost-model picker)")
    ap.add_argument("--fused-merge", action="store_true", help="merge split-K partials inside the attention kernel")
    ap.add_argument("--plan-cus", type=int, default=None,
                    help="attention workloads: plan for this many CUs (workgroups of the streaming kernel)")
    ap.add_argument("--plan-opts", default="",
                    help="attention workloads: comma-separated planner switches (no_tail, tail_role, no_tail_role, no_regs, "
                         "no_wide, no_wide256, tile_kernel)")
    ap.add_argument("--row-blocks", default="auto", choices=["auto", "on", "off"],
                    help="attention: the row-block kernel (one launch, no partials) forced on or off")
    ap.add_argument("--selection", default="vanilla", choices=["vanilla", "diverse"],
                    help="e2e: beam selection (vanilla, or diverse beam search with 4 groups)")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-graphs", action="store_true", help="e2e: launch every op eagerly (no HIP graphs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-flat", action="store_true", help="e2e: skip the flat-strategy run of the same prompts")
    ap.add_argument("--picker-costs", default="mi355x", choices=["mi355x", "fasttree"],
                    help="e2e tree / auto: edge decisions by the MI355X-fitted costs or the reference's FastTree model")
    ap.add_argument("--verbose", action="store_true")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------- attention
def attention_traffic(name, args):
    """HBM bytes per launch measured by rocprofv3 counter runs of the same
    workload (profiles/attn_traffic.json, cascade plans with default options),
    or (None, None)."""
    if args.strategy != "cascade" or args.plan_opts or args.plan_cus or args.fused_merge or args.row_blocks != "auto":
        return None, None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "attn_traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(f"attn-{name}:cascade")
    except (OSError, ValueError):
        return None, None
    if not entry:
        return None, None
    return int(entry["traffic_bytes_per_launch"]), entry["source"]


def attention_workload(args):
    import torch
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper, MultiLevelCascadeAttentionWrapper
    from beam_engine_amd.workloads import BUILDERS

    wl = BUILDERS[args.workload.split("-", 1)[1]]()
    dtype = torch.float32 if wl.name == "c1" else torch.bfloat16
    es = 4 if dtype == torch.float32 else 2
    steps = args.steps or 20
    warmup = 5 if args.warmup is None else args.warmup
    L = args.layers
    dev = torch.device("cuda")
    torch.manual_seed(0)
    scale = 1.0 / math.sqrt(wl.d)
    log(f"{wl.name}: {wl.note}; {wl.num_pages} pages x {L} layers")
    kv = [torch.randn((wl.num_pages, 2, wl.page, wl.hkv, wl.d), device=dev, dtype=dtype).mul_(scale) for _ in range(L)]
    qs = [torch.randn((wl.num_queries, wl.hq, wl.d), device=dev, dtype=dtype).mul_(scale) for _ in range(L)]
    outs = [torch.empty_like(q) for q in qs]
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    def tune(w):
        w._fused_merge = args.fused_merge
        w._rows = {"auto": None, "on": True, "off": False}[args.row_blocks]
        w._num_cus = args.plan_cus
        for opt in filter(None, args.plan_opts.split(",")):
            if opt not in ("no_tail", "tail_role", "no_tail_role", "no_regs", "no_wide", "no_wide256", "tile_kernel"):
                raise SystemExit(f"unknown --plan-opts entry {opt!r}")
            if opt == "no_tail_role":
                w._tail_role = False
            else:
                setattr(w, "_" + opt, True)
        return w
    if args.strategy == "cascade":
        w = tune(MultiLevelCascadeAttentionWrapper(len(wl.levels[0]), ws))
        w.plan(*wl.levels, wl.hq, wl.hkv, wl.d, wl.page, q_data_type=dtype)
        alg_kv = w.stats.kv_bytes
    elif args.strategy == "flat":
        w = tune(BatchDecodeWithPagedKVCacheWrapper(ws))
        w.plan(*wl.flat, wl.hq, wl.hkv, wl.d, wl.page, q_data_type=dtype)
        alg_kv = sum(wl.tokens_per_query) * wl.hkv * wl.d * es * 2     # flat scored by its own path bytes
    else:
        # the exact path decompositions of the workload's segment tree
        lv = wl.decomposition(args.strategy)
        w = tune(MultiLevelCascadeAttentionWrapper(len(lv), ws))
        w.plan([l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv], [l[3] for l in lv], wl.hq, wl.hkv, wl.d,
               wl.page, q_data_type=dtype)
        alg_kv = w.stats.kv_bytes
    st = w.stats
    alg = alg_kv + st.qo_bytes
    for _ in range(warmup):
        for l in range(L):
            w.run(qs[l], kv[l], out=outs[l])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps * L)]
    loop = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for r in range(steps):
        loop[r][0].record(stream)
        for l in range(L):
            s, e = evs[r * L + l]
            s.record(stream)
            w.run(qs[l], kv[l], out=outs[l])
            e.record(stream)
        loop[r][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) * 1e3 for s, e in evs]            # us per launch
    mean_us = sum(per) / len(per)
    med_us = statistics.median(per)
    layer_us = statistics.median([a.elapsed_time(b) * 1e3 / L for a, b in loop])
    gbs = alg / (mean_us * 1e-6) / 1e9
    tflops = st.flops / (mean_us * 1e-6) / 1e12
    traffic, traffic_src = attention_traffic(wl.name, args)
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
            "kernel": f"attn_{st.kernel}_kernel" + ("" if st.num_merge == 0 or args.fused_merge else
                                                    " + tail_merge_kernel" if st.kernel == "stream" else " + merge_kernel"),
            "bytes_per_launch": alg, "mean_launch_us": round(mean_us, 2), "median_launch_us": round(med_us, 2),
            "tflops": round(tflops, 2), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4)}
    result = {
        "metric": "decode attention HBM GB/s (algorithmic bytes / kernel time)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(layer_us * L / 1e3, 4), "higher_is_better": True, "scaling": "strong",
        "vs_baseline": None, "dtype": "f32" if es == 4 else "bf16", "data": "synthetic N(0,1)/sqrt(D)",
        "config": {"workload": f"attention {wl.name} {args.strategy}", "shape": wl.note, "layers": L,
                   "items": st.num_items, "chunk_tokens": st.chunk_tokens, "merge_rows": st.num_part_rows,
                   "fused_merge": bool(args.fused_merge), "per_layer_us": round(layer_us, 2),
                   "wall_s": round(wall, 3)},
        "roofline": roof,
    }
    return result, wl


def prefill_workload(args):
    """Causal paged prefill attention at the e2e prompt shape: 8 requests x
    1024 tokens, 32 / 8 heads, head_dim 128, bf16, page 16, over 32 distinct
    per-layer caches.  Compute-bound: value = TFLOP/s (4 D Hq sum of visible
    tokens per launch), roofline against the bf16 MFMA peak."""
    import torch
    from beam_engine_amd import BatchPrefillWithPagedKVCacheWrapper
    r, s, hq, hkv, d, ps = 8, 1024, 32, 8, 128, 16
    steps = args.steps or 10
    warmup = 3 if args.warmup is None else args.warmup
    L = args.layers
    dev = torch.device("cuda")
    torch.manual_seed(0)
    npg = s // ps
    sc = 1.0 / math.sqrt(d)
    kv = [torch.randn((r * npg, 2, ps, hkv, d), device=dev, dtype=torch.bfloat16).mul_(sc) for _ in range(L)]
    qs = [torch.randn((r * s, hq, d), device=dev, dtype=torch.bfloat16).mul_(sc) for _ in range(L)]
    outs = [torch.empty_like(q) for q in qs]
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    w = BatchPrefillWithPagedKVCacheWrapper(ws)
    w.plan([i * s for i in range(r + 1)], [i * npg for i in range(r + 1)], list(range(r * npg)), [ps] * r,
           hq, hkv, d, ps, causal=True, q_data_type=torch.bfloat16)
    st = w.stats
    for _ in range(warmup):
        for l in range(L):
            w.run(qs[l], kv[l], out=outs[l])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps * L)]
    for i in range(steps * L):
        evs[i][0].record(stream)
        w.run(qs[i % L], kv[i % L], out=outs[i % L])
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    mean_us = sum(a.elapsed_time(b) for a, b in evs) * 1e3 / len(evs)
    tflops = st.flops / (mean_us * 1e-6) / 1e12
    gbs = st.bytes / (mean_us * 1e-6) / 1e9
    return {
        "metric": "prefill attention TFLOP/s (causal, paged)", "value": round(tflops, 2), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(mean_us * L / 1e3, 4),
        "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1)/sqrt(D)",
        "config": {"workload": "prefill attention, 8 x 1024-token prompts, Llama-3-8B layer shape, causal",
                   "layers": L, "items": st.num_items, "flops_per_launch": st.flops},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": f"attn_{st.kernel}_kernel" + (" + tail_merge_kernel" if st.kernel == "stream" else
                                                             " + merge_kernel"),
                     "mean_launch_us": round(mean_us, 2),
                     "hbm_gbs": round(gbs, 1)},
    }


def topk_workload(args):
    """Beam selection (log_softmax + row top-2B + per-request top-B) on the GPU:
    ``topk`` = the e2e step (8 requests x beam 16 rows of a 128256 vocabulary,
    bf16 logits), ``topk-c1`` = config 1 (one request, beam 4, 32000, fp32).
    Value = logits bytes / time (each logit is needed once); the CPU baseline
    is the oracle's float64 selection on the same logits."""
    import numpy as np
    import torch
    from beam_engine_amd.selection import beam_topk
    c1 = args.workload == "topk-c1"
    reqs, beam, vocab = (1, 4, 32000) if c1 else (8, 16, 128256)
    dtype = torch.float32 if c1 else torch.bfloat16
    n = reqs * beam
    k = 2 * beam
    steps = args.steps or 50
    warmup = 5 if args.warmup is None else args.warmup
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(0)
    # 32 distinct logit sets (the e2e working set is one [N, V] per step)
    sets = [torch.randn((n, vocab), generator=g).to(dtype).to(dev) for _ in range(8)]
    # parent scores resident on the device, as the decode loop keeps them (a CPU
    # tensor would add a synchronous host-to-device copy to every call)
    parents = torch.from_numpy(-np.random.default_rng(0).random(n)).to(dev)
    rows = [beam] * reqs
    for i in range(warmup):
        beam_topk(sets[i % 8], k, parents, beam, request_rows=rows)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        beam_topk(sets[i % 8], k, parents, beam, request_rows=rows)
    t1.record(stream)
    torch.cuda.synchronize()
    mean_us = t0.elapsed_time(t1) * 1e3 / steps
    byts = n * vocab * (4 if c1 else 2)
    gbs = byts / (mean_us * 1e-6) / 1e9
    result = {
        "metric": "beam selection GB/s (logits bytes / time)", "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(mean_us / 1e3, 4), "higher_is_better": True,
        "scaling": "strong", "vs_baseline": None, "dtype": "f32" if c1 else "bf16", "data": "synthetic N(0,1) logits",
        "config": {"workload": f"beam selection, {reqs} request(s) x beam {beam}, vocab {vocab}, k {k}"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "topk_units16 + topk_rows16 kernels (16-bit logits)",
                     "bytes_per_launch": byts, "mean_launch_us": round(mean_us, 2)},
    }
    if not args.no_cpu_baseline:
        from oracle import topk as ot
        x = sets[0][:beam].float().cpu().numpy()
        t0 = time.perf_counter()
        ot.beam_step(x, parents[:beam].cpu().tolist(), beam, "float32" if c1 else "bfloat16")
        dt = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(beam * vocab * (4 if c1 else 2) / dt / 1e9, 4), "unit": "GB/s",
                                  "cores": len(os.sched_getaffinity(0)), "kind": "port",
                                  "sample": f"oracle selection (numpy float64) of one request ({beam} rows): {dt:.2f} s"}
    return result


def read_ceiling_workload(args):
    """The read ceiling the attention roofline is read against: one launch of
    a plain read kernel (``be_read_probe``) over one north-star layer's K/V
    (3072 pages of [2, 16, 8, 128] bf16 = 201 MB) per call, 32 distinct layers,
    HIP events around each launch as the attention workloads time theirs.
    Two access patterns -- the layer as one contiguous range, and one KV head's
    256-byte rows at a 2 KB stride at a time (the decode kernels' pattern) --
    over a sweep of grid sizes; value = the best per-launch GB/s."""
    import torch
    from beam_engine_amd import _lib
    lib = _lib.load()
    P, page, hkv, d = 3072, 16, 8, 128
    L = args.layers
    steps = args.steps or 10
    warmup = 3 if args.warmup is None else args.warmup
    dev = torch.device("cuda")
    layers = [torch.empty((P, 2, page, hkv, d), dtype=torch.bfloat16, device=dev).fill_(0.5) for _ in range(L)]
    nbytes = layers[0].numel() * 2
    sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    patterns = {"contiguous": (nbytes // 256, nbytes // 256, 256, 0, 256),
                "per KV head": (P * 2 * page * hkv, P * 2 * page, hkv * d * 2, d * 2, d * 2)}
    results = []
    for name, (rows, inner, istr, ostr, rb) in patterns.items():
        for grid in (256, 1024, 2048, 4096, 8192, 16384):
            def launch(l):
                _lib.check(lib.be_read_probe(layers[l].data_ptr(), rows, inner, istr, ostr, rb, sink.data_ptr(),
                                             grid, stream.cuda_stream), "read probe")
            for _ in range(warmup):
                for l in range(L):
                    launch(l)
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(steps * L)]
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(evs):
                a.record(stream)
                launch(i % L)
                b.record(stream)
            torch.cuda.synchronize()
            us = sum(a.elapsed_time(b) for a, b in evs) * 1e3 / len(evs)
            results.append({"pattern": name, "grid": grid, "us": round(us, 2),
                            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
            log(f"read probe {name} grid {grid}: {us:.2f} us per launch, {results[-1]['gbs']} GB/s")
    best = max(results, key=lambda r: r["gbs"])
    return {
        "metric": "HBM read ceiling GB/s (one launch over one north-star layer's K/V)", "value": best["gbs"],
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(best["us"] * L / 1e3, 4), "higher_is_better": True, "scaling": "strong",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "read ceiling: be_read_probe over 3072 pages x [2, 16, 8, 128] bf16 (201 MB) per launch",
                   "layers": L, "bytes_per_launch": nbytes, "sweep": results},
        "roofline": {"bound": "hbm", "achieved": best["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(best["gbs"] / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "read_probe_kernel",
                     "bytes_per_launch": nbytes, "mean_launch_us": best["us"]},
    }


# ---------------------------------------------------------------------- CPU baseline
def cpu_baseline_attention(wl, alg_bytes):
    """The CPU restatement (torch float32 paged gather, per-level softmax
    attention, log-sum-exp merge: the reference's CPU path) on one layer of the
    same workload, in GB/s of the same algorithmic bytes."""
    import torch
    from bench_e2e import cpu_model
    from oracle import attention as oa
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    kv = torch.randn((wl.num_pages, 2, wl.page, wl.hkv, wl.d), generator=g)
    q = torch.randn((wl.num_queries, wl.hq, wl.d), generator=g)
    t0 = time.perf_counter()
    oa.cascade_attention_torch(q, kv, *wl.levels, wl.page, wl.d ** -0.5)
    dt = time.perf_counter() - t0
    gbs = alg_bytes / dt / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port", "cpu": cpu_model(),
            "sample": f"torch float32 cascade attention on the host ({threads} threads) over all "
                      f"{wl.num_queries} queries of one layer: {dt:.2f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: bench.py --gpus N with N > 1 is not "
                                   "supported (sharding across GPUs is designed, not built)"}))
        return 2
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        return 1
    if args.workload.startswith("topk"):
        print(json.dumps(topk_workload(args)), flush=True)
        return 0
    if args.workload == "read-ns":
        print(json.dumps(read_ceiling_workload(args)), flush=True)
        return 0
    if args.workload == "attn-prefill":
        print(json.dumps(prefill_workload(args)), flush=True)
        return 0
    if args.workload.startswith("attn-"):
        result, wl = attention_workload(args)
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline_attention(wl, result["roofline"]["bytes_per_launch"])
    else:
        from bench_e2e import run_e2e_bench
        result = run_e2e_bench(args)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
