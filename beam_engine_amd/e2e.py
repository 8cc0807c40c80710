"""End-to-end beam-search benchmark (the 8-request, beam-16 Llama-3-8B workload).

Random-init Llama-3-8B-shaped decoder (32 layers, hidden 4096, 32/8 heads,
head_dim 128, FFN 14336, vocab 128256, bf16 weights ~ N(0, 0.02)), 8 requests
with random 1024-token prompts, beam width 16, length penalty 1.0.  A bench
step is one decode step of all 8 x 16 = 128 candidates; tokens/s = 128 x
timed steps / timed wall time (prefill excluded).

In every timed decode step one decode-attention launch -- that of layer
(step mod 32), so every layer and every step of the run is sampled alike --
is bracketed by two HIP events on the launch stream (events around all 32
launches of a step cost about 4% of the step).  The roofline reports the plan's
algorithmic bytes against the mean duration of both kernels of a launch
together: with the streaming kernel, short groups are attended inside the
tail-and-merge kernel, so the pair is the unit that reads the plan's bytes
(each kernel's own share is in the rocprofv3 summaries).
"""

from __future__ import annotations

import json
import math
import os
import platform
import sys
import time

import numpy as np
import torch

from .generator import BatchedBeamSearch
from .llama import LlamaConfig, LlamaDecoder
from .page_table import PageTable

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[e2e] {msg}", file=sys.stderr, flush=True)


class AttnTimer:
    """Events start -> attention kernel, merge kernel -> end around the launch
    of layer (step mod layers) of every step."""

    def __init__(self, kind: str, hkv: int, d: int, es: int, layers: int):
        self.records = []      # (start, end, algorithmic bytes, flops)
        self.kind = kind
        self.kernels = set()   # attention kernels the plans used
        self.hkv, self.d, self.es = hkv, d, es
        self.layers = layers
        self.step = -1

    def __call__(self, layer, run_fn, wrapper):
        if layer == 0:
            self.step += 1
        if layer != self.step % self.layers:
            return run_fn(None)
        st = wrapper.stats
        self.kernels.add(st.kernel)
        if self.kind == "flat":
            # the flat strategy is scored by its own traffic: every query's whole path
            hq = wrapper._info.num_qo_heads
            kv = int(round(st.flops / (4.0 * self.d * hq))) * self.hkv * self.d * self.es * 2
        else:
            kv = st.kv_bytes
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        out = run_fn(None)
        e.record()
        self.records.append((s, e, kv + st.qo_bytes, st.flops))
        return out


def use_tuned_gemms(path: str = None) -> bool:
    """Use the TunableOp results file written by ``beam_engine_amd.tune_gemms``
    (the decode GEMMs' library solutions, timed on this GPU) with tuning off;
    shapes not in the file keep the library's default choice.  Returns False
    (and leaves TunableOp off) when the file is missing or was written for
    another GPU or library version."""
    from .tune_gemms import DEFAULT_FILE
    path = path or DEFAULT_FILE
    if not os.path.exists(path):
        return False
    tun = torch.cuda.tunable
    try:
        tun.enable(True)
        tun.tuning_enable(False)
        tun.record_untuned_enable(False)
        ok = bool(tun.read_file(path))
    except Exception as e:               # validator mismatch and the like
        log(f"tuned GEMM file not used: {e}")
        ok = False
    if not ok:
        tun.enable(False)
    return ok


def run_e2e(steps: int, warmup: int, kernel_type: str = "cascade", n_req: int = 8, beam: int = 16,
            prompt_len: int = 1024, cfg: LlamaConfig = None, seed: int = 0, time_attention: bool = True,
            max_pages: int = 8192, graphs: bool = True, tuned_gemms: bool = True, selection: str = "vanilla"):
    cfg = cfg or LlamaConfig.llama3_8b()
    dev = torch.device("cuda")
    tuned = use_tuned_gemms() if tuned_gemms else False
    log(f"decode GEMMs: {'TunableOp results file' if tuned else 'library defaults'}")
    t0 = time.perf_counter()
    model = LlamaDecoder(cfg, dev, torch.bfloat16, seed)
    pt = PageTable(cfg.num_hidden_layers, page_size=16, max_num_pages=max_pages, head_num=cfg.num_key_value_heads,
                   head_dim=cfg.head_dim, device=dev, store_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    log(f"model {cfg.num_params() / 1e9:.2f} B params + {pt.kv_pool.numel() * 2 / 2**30:.1f} GiB KV pool "
        f"ready in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(seed)
    prompts = rng.integers(0, cfg.vocab_size, size=(n_req, prompt_len)).tolist()
    strategy = None
    if selection == "diverse":
        from .beam_strategy import DiverseBeamSearchStrategy
        strategy = DiverseBeamSearchStrategy(num_groups=4, diversity_penalty=0.5)
    gen = BatchedBeamSearch(model, pt, beam, strategy=strategy, kernel_type=kernel_type, graphs=graphs)
    timer = AttnTimer(kernel_type, cfg.num_key_value_heads, cfg.head_dim, 2, cfg.num_hidden_layers) \
        if time_attention else None
    t0 = time.perf_counter()
    gen.prefill(prompts)
    torch.cuda.synchronize()
    log(f"prefill {n_req} x {prompt_len} in {time.perf_counter() - t0:.1f} s")
    for _ in range(warmup):
        gen.step()
    torch.cuda.synchronize()
    log(f"{warmup} warmup steps done")
    gen.attn_timer = timer
    t0 = time.perf_counter()
    for i in range(steps):
        gen.step()
        if (i + 1) % 50 == 0:
            log(f"step {i + 1}/{steps}")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return gen, timer, wall, model, pt


def summarize_attention(timer: AttnTimer):
    pair_us, byts, flops = [], 0, 0.0
    for s, e, b, f in timer.records:
        pair_us.append(s.elapsed_time(e) * 1e3)
        byts += b
        flops += f
    n = len(pair_us)
    tot = sum(pair_us)
    gbs = byts / (tot * 1e-6) / 1e9
    return {
        "launches": n, "mean_pair_us": tot / n, "bytes_per_launch": byts / n, "gbs": gbs,
        "tflops": flops / (tot * 1e-6) / 1e12,
    }


def cpu_baseline_e2e(gen: BatchedBeamSearch, budget_s: float = 20.0):
    """The CPU oracle on a bounded sample of the same workload: one decode
    step's hot path at the run's final beam state -- cascade attention of one
    layer (numpy float64 over the state's real pages and index arrays; the 32
    layers are extrapolated from it), the cascade metadata restatement, and the
    token selection of all 8 requests (float64 pool sort).  Model GEMMs are not
    part of the path and are not timed."""
    from oracle import attention as oa
    from oracle import topk as ot
    st = gen.state
    cfg = gen.model.cfg
    threads = len(os.sched_getaffinity(0))
    levels = st._cascade_lists()
    lv = ([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels])
    n = len(st.candidates)
    used = sorted({p for l in lv[2] for p in l})
    remap = {p: i for i, p in enumerate(used)}
    kv = gen.pt.kv_cache_at_layer[0][torch.tensor(used, device=gen.pt.device)].float().cpu().numpy()
    lv_remap = (lv[0], lv[1], [[remap[p] for p in l] for l in lv[2]], lv[3])
    q = np.random.default_rng(1).standard_normal((n, cfg.num_attention_heads, cfg.head_dim)).astype(np.float32)
    t0 = time.perf_counter()
    oa.cascade_attention(q, kv, *lv_remap, gen.pt.page_size, cfg.head_dim ** -0.5)
    t_attn = time.perf_counter() - t0
    # metadata: the oracle's get_cascade_input over an equivalent trie
    from oracle.beam_state import OracleAllocator, OracleBeamState, ONode, OCand
    o = OracleBeamState(gen.beam_size, OracleAllocator(gen.pt.max_num_pages, gen.pt.page_size))
    memo = {}

    def conv(node):
        if id(node) in memo:
            return memo[id(node)]
        par = conv(node.parent) if node.parent is not None else None
        on = ONode(list(node.tokens), node.page_id, par)
        memo[id(node)] = on
        return on
    o.candidates = [OCand(conv(c.trie_node), c.score) for c in st.candidates]
    t0 = time.perf_counter()
    o.get_cascade_input()
    t_meta = time.perf_counter() - t0
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((gen.beam_size, cfg.vocab_size)).astype(np.float32)
    t0 = time.perf_counter()
    ot.beam_step(logits, [0.0] * gen.beam_size, gen.beam_size, "bfloat16")
    t_sel = (time.perf_counter() - t0) * (n // gen.beam_size)
    step_s = t_attn * cfg.num_hidden_layers + t_meta + t_sel
    return {"value": round(n / step_s, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"one decode step of the hot path at the final beam state ({n} candidates): oracle cascade "
                       f"attention of 1 layer {t_attn:.2f} s x {cfg.num_hidden_layers} layers (extrapolated), "
                       f"cascade metadata {t_meta * 1e3:.1f} ms, selection of {n // gen.beam_size} requests "
                       f"{t_sel:.2f} s; model GEMMs excluded; numpy float64, {threads} BLAS threads, cpu "
                       f"{platform.processor() or platform.machine()}")}


def profiled_traffic(kind: str, steps: int):
    """HBM traffic per attention launch measured by rocprofv3 counter runs of
    the default bench command (profiles/e2e_llama8b_beam16_cascade_traffic.*),
    or None for a run that is not that command."""
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles",
                        "e2e_llama8b_beam16_cascade_traffic.json")
    if kind != "cascade" or steps != 250 or not os.path.exists(path):
        return None, None
    with open(path) as f:
        data = json.load(f)
    if data.get("kernel") != "attn_stream_kernel + tail_merge_kernel":
        return None, None          # measured for another kernel pair
    return int(data["traffic_bytes_per_launch"]), "profiles/e2e_llama8b_beam16_cascade_traffic.md"


def run_e2e_bench(args):
    steps = args.steps if args.steps is not None else 250
    warmup = args.warmup if args.warmup is not None else 5
    kind = args.strategy
    selection = getattr(args, "selection", "vanilla")
    gen, timer, wall, model, pt = run_e2e(steps, warmup, kind, graphs=not getattr(args, "no_graphs", False),
                                          selection=selection)
    n = len(gen.state.candidates)
    tok_s = n * steps / wall
    traffic, traffic_src = profiled_traffic(kind, steps) if selection == "vanilla" else (None, None)
    att = summarize_attention(timer)
    log(f"{kind}: {steps} steps in {wall:.2f} s -> {tok_s:.1f} tokens/s; attention {att['mean_pair_us']:.1f} us "
        f"per layer (both kernels), {att['gbs']:.0f} GB/s")
    result = {
        "metric": "beam-decode tokens/sec @ beam 16 (1 GPU)",
        "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(wall / steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02), random token-id prompts",
        "config": {"workload": f"e2e beam search, Llama-3-8B shape, {kind} attention"
                               + (", diverse beam search (4 groups, Hamming penalty 0.5)" if selection == "diverse" else ""),
                   "requests": 8, "beam": 16, "prompt_len": 1024, "decode_steps": warmup + steps,
                   "layers": model.cfg.num_hidden_layers, "page_size": 16, "length_penalty": 1.0,
                   "per_request_tokens_per_s": round(tok_s / 8, 2),
                   **({"picker_choices": {k: gen.picker.history.count(k) for k in sorted(set(gen.picker.history))}}
                      if kind == "auto" and gen.picker is not None else {})},
        "roofline": {"bound": "hbm", "achieved": round(att["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(att["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": " / ".join(f"attn_{k}_kernel" for k in sorted(timer.kernels)) +
                               (" + tail_merge_kernel" if timer.kernels == {"stream"} else " + merge_kernel") +
                               " (decode attention: both kernels of a launch)",
                     "timed_launches": att["launches"],
                     "timed_sample": "the launch of layer (step mod 32) in every timed step",
                     "bytes_per_launch": round(att["bytes_per_launch"]),
                     "mean_launch_us": round(att["mean_pair_us"], 2),
                     "attention_tflops": round(att["tflops"], 2)},
    }
    if not getattr(args, "no_cpu_baseline", False):
        result["cpu_baseline"] = cpu_baseline_e2e(gen)
    return result
