"""End-to-end beam-search benchmark harness (benchmark config 4), used by bench.py.

Random-init Llama-3-8B-shaped decoder (32 layers, hidden 4096, 32/8 heads,
head_dim 128, FFN 14336, vocab 128256, bf16 weights ~ N(0, 0.02)), 8 requests
with random 1024-token prompts, beam width 16, length penalty 1.0, and a
generation of 256 decode steps, as config 4 specifies (the reference decodes
to ``max_length``, beam.py:145).  tokens/s = 128 candidate tokens per step /
step time; prefill is excluded.

``--steps K`` steps of the 256 are timed, spread evenly over the generation
after ``--warmup W`` untimed steps (step W + floor(i (256 - W) / K) for
i < K), each bracketed by a device synchronisation on both sides, so the
sample covers short and long beam suffixes alike.  The whole 256-step decode
is also timed (``generation_tokens_per_s``).  The flat strategy runs the same
prompts through the same model in the same process, for the ratio.

In every timed step one decode-attention launch -- that of layer (step mod
32) -- is bracketed by two HIP events on the launch stream: inside the step
when its attention runs eagerly, or, when the step ran as one HIP graph,
launched again right after the step (outside its timing) with the step's
plan, queries and cache.  The roofline reports the plan's algorithmic bytes
against the mean duration of both kernels of a launch together.

The model's GEMMs are library calls outside the hot path; their library
solutions come from the TunableOp results file ``bench_gemms.csv`` (timed
with weights streaming from HBM by ``python bench_e2e.py --tune-gemms``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

from beam_engine_amd.generator import BatchedBeamSearch
from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
from beam_engine_amd.page_table import PageTable

ROOT = os.path.dirname(os.path.abspath(__file__))
GEMM_FILE = os.path.join(ROOT, "bench_gemms.csv")
HBM_PEAK_GBS = 8000.0
DECODE_STEPS = 256          # config 4: 256 generated tokens
REQUESTS, BEAM, PROMPT = 8, 16, 1024

# (N, K) of y[M, N] = x[M, K] W[N, K]^T for the five decode GEMMs
GEMM_SHAPES = {"qkv": (6144, 4096), "o_proj": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336),
               "lm_head": (128256, 4096)}


def log(msg):
    print(f"[e2e] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------- library GEMMs
def use_tuned_gemms(path: str = GEMM_FILE) -> bool:
    """Load the TunableOp results file (tuning off); shapes not in the file keep
    the library's default.  False (TunableOp left off) when the file is
    missing or was written for another GPU or library version."""
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


def tune_gemms(path: str = GEMM_FILE, m: int = REQUESTS * BEAM) -> None:
    """Time every library solution of the five decode GEMM shapes with
    TunableOp, rotating over more weight copies than the 256 MB Infinity Cache
    holds, and write the winners to ``path``."""
    import torch.nn.functional as F
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.record_untuned_enable(False)
    tun.set_rotating_buffer_size(1024)
    tun.set_max_tuning_duration(200)
    tun.set_filename(path)
    dev = torch.device("cuda")
    for name, (n, k) in GEMM_SHAPES.items():
        x = torch.randn(m, k, device=dev, dtype=torch.bfloat16)
        w = torch.randn(n, k, device=dev, dtype=torch.bfloat16) * 0.02
        F.linear(x, w)
        torch.cuda.synchronize()
        log(f"tuned {name}: [{m}, {k}] x [{n}, {k}]^T")
    write = getattr(torch._C, "_cuda_tunableop_write_file", None)
    if write is not None:
        write(path)


# ---------------------------------------------------------------------- attention timing
class AttnTimer:
    """Events start -> attention kernel, merge kernel -> end around the launch
    of layer (step mod layers) of every timed step."""

    def __init__(self, kind: str, hkv: int, d: int, es: int, layers: int):
        self.records = []      # (start, end, algorithmic bytes, flops)
        self.kind = kind
        self.kernels = set()   # attention kernels the plans used
        self.hkv, self.d, self.es = hkv, d, es
        self.layers = layers
        self.layer = -1        # layer to time in the current step (-1: none)

    def _bytes(self, wrapper):
        st = wrapper.stats
        self.kernels.add(st.kernel)
        if self.kind == "flat":
            # the flat strategy is scored by its own traffic: every query's whole path
            hq = wrapper._info.num_qo_heads
            kv = int(round(st.flops / (4.0 * self.d * hq))) * self.hkv * self.d * self.es * 2
        else:
            kv = st.kv_bytes
        return kv + st.qo_bytes, st.flops

    def __call__(self, layer, run_fn, wrapper):
        if layer != self.layer:
            return run_fn(None)
        byts, flops = self._bytes(wrapper)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        out = run_fn(None)
        e.record()
        self.records.append((s, e, byts, flops))
        return out

    def after_step_graph(self, gen, layer):
        """A step that ran as one graph: launch that layer's attention again,
        right after the step and outside its timing, with the step's plan,
        queries and cache (the same launch), into a scratch output."""
        w = gen.last_attn
        q = gen._gd.step_q[layer]
        if getattr(self, "_scratch", None) is None or self._scratch.shape != q.shape:
            self._scratch = torch.empty_like(q)
        byts, flops = self._bytes(w)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # the device idles after the step: a short spin keeps it busy while the
        # host enqueues the events and the launch, so the bracket holds the two
        # kernels and not the host's launch latency
        torch.cuda._sleep(200000)
        s.record()
        w.run(q, gen.pt.kv_cache_at_layer[layer], out=self._scratch)
        e.record()
        self.records.append((s, e, byts, flops))

    def summary(self):
        us, byts, flops = [], 0, 0.0
        for s, e, b, f in self.records:
            us.append(s.elapsed_time(e) * 1e3)
            byts += b
            flops += f
        tot = sum(us)
        n = len(us)
        return {"launches": n, "mean_pair_us": tot / n, "bytes_per_launch": byts / n,
                "gbs": byts / (tot * 1e-6) / 1e9, "tflops": flops / (tot * 1e-6) / 1e12}


def timed_indices(steps: int, warmup: int, total: int = DECODE_STEPS):
    """``steps`` step indices spread evenly over [warmup, total)."""
    warmup = min(max(warmup, 0), total - 1)
    steps = max(1, min(steps, total - warmup))
    return [warmup + (i * (total - warmup)) // steps for i in range(steps)]


# ---------------------------------------------------------------------- one generation
def generate(model, cfg, prompts, kind: str, timed, graphs: bool = True, selection: str = "vanilla",
             max_pages: int = 8192, picker_costs: str = "mi355x"):
    """Prefill + DECODE_STEPS decode steps; the steps in ``timed`` are each
    bracketed by synchronisations.  Returns (gen, per-step seconds of the timed
    steps, whole-decode seconds, timer)."""
    dev = model.device
    pt = PageTable(cfg.num_hidden_layers, page_size=16, max_num_pages=max_pages, head_num=cfg.num_key_value_heads,
                   head_dim=cfg.head_dim, device=dev, store_dtype=torch.bfloat16)
    strategy = None
    if selection == "diverse":
        from beam_engine_amd.beam_strategy import DiverseBeamSearchStrategy
        strategy = DiverseBeamSearchStrategy(num_groups=4, diversity_penalty=0.5)
    gen = BatchedBeamSearch(model, pt, BEAM, strategy=strategy, kernel_type=kind, graphs=graphs,
                            picker_costs=picker_costs)
    timer = AttnTimer(kind, cfg.num_key_value_heads, cfg.head_dim, 2, cfg.num_hidden_layers)
    gen.attn_timer = timer
    t0 = time.perf_counter()
    gen.prefill(prompts)
    torch.cuda.synchronize()
    log(f"{kind}: prefill {len(prompts)} x {len(prompts[0])} in {time.perf_counter() - t0:.1f} s")
    gen.prepare_graphs()                 # capture time is set-up, not decode time
    torch.cuda.synchronize()
    timed = set(timed)
    per_step = []
    torch.cuda.synchronize()
    t_all = time.perf_counter()
    for i in range(DECODE_STEPS):
        if i in timed:
            timer.layer = i % cfg.num_hidden_layers
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            gen.step()
            torch.cuda.synchronize()
            per_step.append(time.perf_counter() - t0)
            if gen.step_graphed:
                timer.after_step_graph(gen, i % cfg.num_hidden_layers)
            timer.layer = -1
        else:
            gen.step()
        if (i + 1) % 64 == 0:
            log(f"{kind}: step {i + 1}/{DECODE_STEPS}")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_all
    return gen, per_step, wall, timer


# ---------------------------------------------------------------------- CPU baseline
def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_baseline_e2e(gen: BatchedBeamSearch, budget_s: float = 25.0):
    """The CPU restatement (oracle/) of the hot path on one decode step at the
    generation's final beam state, in the form the reference's CPU path takes:
    torch float32 cascade attention on the host for every layer (the state's
    real pages and index arrays; layer 0's K/V stand in for each layer's, with
    distinct queries), the cascade metadata restatement, and the vanilla
    selection of all requests (float64 pool sort).  Model GEMMs are not part
    of the path and are not timed.  Layers beyond ``budget_s`` of attention are
    not run and the step time is scaled up from those that ran (reported)."""
    from oracle import attention as oa
    from oracle import topk as ot
    from oracle.beam_state import OCand, ONode, OracleAllocator, OracleBeamState
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    st = gen.state
    cfg = gen.model.cfg
    levels = st._cascade_lists()
    lv = ([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels])
    n = len(st.candidates)
    used = sorted({p for l in lv[2] for p in l})
    remap = {p: i for i, p in enumerate(used)}
    kv = gen.pt.kv_cache_at_layer[0][torch.tensor(used, device=gen.pt.device)].cpu()
    lv_remap = (lv[0], lv[1], [[remap[p] for p in l] for l in lv[2]], lv[3])
    g = torch.Generator().manual_seed(1)
    layers_run = 0
    t0 = time.perf_counter()
    for _ in range(cfg.num_hidden_layers):
        q = torch.randn((n, cfg.num_attention_heads, cfg.head_dim), generator=g)
        oa.cascade_attention_torch(q, kv, *lv_remap, gen.pt.page_size, cfg.head_dim ** -0.5)
        layers_run += 1
        if time.perf_counter() - t0 > budget_s:
            break
    t_attn = (time.perf_counter() - t0) * cfg.num_hidden_layers / layers_run
    # metadata: the oracle's get_cascade_input over the same trie
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
    reqs = n // gen.beam_size
    t_sel = 0.0
    for r in range(reqs):
        logits = rng.standard_normal((gen.beam_size, cfg.vocab_size)).astype(np.float32)
        t0 = time.perf_counter()
        ot.beam_step(logits, [c.score for c in st.candidates[r * gen.beam_size:(r + 1) * gen.beam_size]],
                     gen.beam_size, "bfloat16")
        t_sel += time.perf_counter() - t0
    step_s = t_attn + t_meta + t_sel
    note = "" if layers_run == cfg.num_hidden_layers else \
        f" ({layers_run} of {cfg.num_hidden_layers} layers run, scaled)"
    return {"value": round(n / step_s, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": (f"one decode step of the hot path at the final beam state ({n} candidates, step "
                       f"{DECODE_STEPS}): torch float32 cascade attention on the host, {cfg.num_hidden_layers} "
                       f"layers {t_attn:.2f} s{note}; cascade metadata {t_meta * 1e3:.1f} ms; float64 "
                       f"selection of {reqs} requests {t_sel:.2f} s; model GEMMs excluded; {threads} threads")}


# ---------------------------------------------------------------------- traffic profile
def profiled_traffic(config_key: str):
    """HBM traffic per attention launch measured by rocprofv3 counter runs of
    this workload (profiles/e2e_traffic.json keyed by the workload), or None."""
    path = os.path.join(ROOT, "profiles", "e2e_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        data = json.load(f)
    entry = data.get(config_key)
    if not entry:
        return None, None
    return int(entry["traffic_bytes_per_launch"]), entry["source"]


# ---------------------------------------------------------------------- the bench line
def run_e2e_bench(args):
    steps = args.steps if args.steps is not None else 20
    warmup = args.warmup if args.warmup is not None else 5
    kind = args.strategy
    selection = getattr(args, "selection", "vanilla")
    graphs = not getattr(args, "no_graphs", False)
    cfg = LlamaConfig.llama3_8b()
    if getattr(args, "layers", None) and args.layers != cfg.num_hidden_layers:
        cfg.num_hidden_layers = args.layers
    dev = torch.device("cuda")
    tuned = use_tuned_gemms()
    log(f"decode GEMMs: {'TunableOp results file' if tuned else 'library defaults'}")
    t0 = time.perf_counter()
    model = LlamaDecoder(cfg, dev, torch.bfloat16, 0)
    torch.cuda.synchronize()
    log(f"model {cfg.num_params() / 1e9:.2f} B params ready in {time.perf_counter() - t0:.1f} s")
    prompts = np.random.default_rng(0).integers(0, cfg.vocab_size, size=(REQUESTS, PROMPT)).tolist()
    idx = timed_indices(steps, warmup)
    picker_costs = getattr(args, "picker_costs", "mi355x")

    def one(strategy):
        gen, per, wall, timer = generate(model, cfg, prompts, strategy, idx, graphs, selection,
                                         picker_costs=picker_costs)
        n = REQUESTS * BEAM
        finals = gen.final_sequences()
        res = {"tokens_per_s": n * len(per) / sum(per), "ms_per_step": 1e3 * sum(per) / len(per),
               "generation_tokens_per_s": n * DECODE_STEPS / wall, "generation_s": wall,
               "att": timer.summary(), "kernels": sorted(timer.kernels),
               "final_sequences": sum(len(v) for v in finals.values()),
               "picker": ({k: sum(1 for e in gen.step_log if e["kind"] == k)
                           for k in sorted({e["kind"] for e in gen.step_log})} if strategy == "auto" else None),
               "graphed_steps": gen.graphed_steps}
        log(f"{strategy}: {len(per)} sampled steps -> {res['tokens_per_s']:.1f} tokens/s, whole decode "
            f"{res['generation_tokens_per_s']:.1f} tokens/s; attention {res['att']['mean_pair_us']:.1f} us per "
            f"launch, {res['att']['gbs']:.0f} GB/s")
        return gen, res

    gen, main = one(kind)
    flat = None
    if kind != "flat" and not getattr(args, "no_flat", False):
        keep_gen = gen
        gen = None
        torch.cuda.empty_cache()
        _, flat = one("flat")
        gen = keep_gen
    att = main["att"]
    cfg_key = f"{kind}:{selection}:r{REQUESTS}:b{BEAM}:p{PROMPT}:s{DECODE_STEPS}:L{cfg.num_hidden_layers}"
    traffic, traffic_src = profiled_traffic(cfg_key)
    n = REQUESTS * BEAM
    config = {"workload": f"e2e beam search, Llama-3-8B shape, {kind} attention"
                          + (", diverse beam search (4 groups, Hamming penalty 0.5)" if selection == "diverse"
                             else ""),
              "requests": REQUESTS, "beam": BEAM, "prompt_len": PROMPT, "decode_steps": DECODE_STEPS,
              "timed_steps": f"{len(idx)} of the {DECODE_STEPS} steps, evenly spaced from step {idx[0]}",
              "layers": cfg.num_hidden_layers, "page_size": 16, "length_penalty": 1.0,
              "per_request_tokens_per_s": round(main["tokens_per_s"] / REQUESTS, 2),
              "generation_tokens_per_s": round(main["generation_tokens_per_s"], 1),
              "final_sequences": main["final_sequences"]}
    if main["picker"]:
        config["picker_choices"] = main["picker"]
    if flat is not None:
        config["flat"] = {"tokens_per_s": round(flat["tokens_per_s"], 2), "ms_per_step": round(flat["ms_per_step"], 3),
                          "generation_tokens_per_s": round(flat["generation_tokens_per_s"], 1),
                          "attention_us_per_launch": round(flat["att"]["mean_pair_us"], 2),
                          "attention_gbs": round(flat["att"]["gbs"], 1)}
        config["vs_flat"] = round(main["tokens_per_s"] / flat["tokens_per_s"], 3)
        config["vs_flat_generation"] = round(main["generation_tokens_per_s"] / flat["generation_tokens_per_s"], 3)
    kern = main["kernels"]
    result = {
        "metric": "beam-decode tokens/sec @ beam 16 (1 GPU)",
        "value": round(main["tokens_per_s"], 2), "unit": "tokens/s", "n_gpus": 1, "steps": len(idx),
        "warmup": warmup, "ms_per_step": round(main["ms_per_step"], 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02), random token-id prompts",
        "config": config,
        "roofline": {"bound": "hbm", "achieved": round(att["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(att["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": " / ".join(f"attn_{k}_kernel" for k in kern) +
                               (" + tail_merge_kernel" if kern == ["stream"] else " + merge_kernel") +
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


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--tune-gemms", action="store_true", help="time the decode GEMMs' library solutions")
    ap.add_argument("--out", default=GEMM_FILE)
    a = ap.parse_args()
    if a.tune_gemms:
        tune_gemms(a.out)
