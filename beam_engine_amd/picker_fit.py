"""Fits the picker's kernel costs on the GPU at hand, and tables the picker's
choices against measured times.

``python -m beam_engine_amd.picker_fit [--out FILE]`` times the cascade
wrapper (streaming kernel + tail-and-merge kernel, bf16, head_dim 128, page
16; GQA 4 and 8) on a sweep of level sets -- long groups of 1..16 queries
(one to four 16-row MFMA tiles per KV head), short groups that take the tail
pass, two-level sets whose queries need partial slots, groups long and wide
enough for the planner's 128- and 256-row segments, and the benchmark shapes
themselves -- each over enough distinct per-layer caches to stream from HBM,
and solves a non-negative least-squares fit of

    us per layer = fixed + sum_nt tile_nt * tiles(nt) + seg * segments
                   + slot * extra passes + tail * tail chunks
                   + tile_w128 * wide tiles (128 rows) + tile_w256 * wide tiles (256 rows)
                   + tile_sib * tiles of a group's second and later 64-row query tiles

The features are the cost model's own counts (``picker.plan_cost`` under a
unit cost per term), so the fit prices exactly what ``picker.CostModel``
prices.  Prints the fitted ``KernelCosts`` and the per-configuration
residuals; ``--out`` writes them as JSON.

``--table`` times every decomposition the picker chooses among (flat, split,
tree with the fitted edge model, tree with FastTree's, and the reference's
cascade levels) at the benchmark shapes (configs 2, 3 and 5, the north-star
shape, a config-4 decode step) and prints measured and modelled microseconds
per layer with the picker's choice.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import fields, replace

import numpy as np

from .picker import MI355X, CostModel, KernelCosts, StrategyPicker, plan_cost

D, PAGE = 128, 16
TERMS = ("fixed", "tile_nt0", "tile_nt1", "tile_nt2", "tile_nt3", "seg", "slot", "tail", "tile_w128", "tile_w256",
         "tile_sib")


def levels_of(spec):
    """spec: list of levels, each a list of (queries, tokens) groups in query
    order; every level covers the same queries.  Returns (levels, pages)."""
    page = 0
    out = []
    for groups in spec:
        qo, kvp, kvi, lpl = [0], [0], [], []
        for nq, tok in groups:
            npg = max(1, -(-tok // PAGE))
            kvi.extend(range(page, page + npg))
            page += npg
            kvp.append(len(kvi))
            lpl.append(tok - (npg - 1) * PAGE)
            qo.append(qo[-1] + nq)
        out.append((qo, kvp, kvi, lpl))
    return out, page


def _unit(term: str) -> KernelCosts:
    zero = dict(tile_nt=(0.0, 0.0, 0.0, 0.0), seg=0.0, slot=0.0, tail=0.0, fixed=0.0, tile_w128=0.0, tile_w256=0.0,
                tile_sib=0.0)
    if term.startswith("tile_nt"):
        t = [0.0] * 4
        t[int(term[-1])] = 1.0
        zero["tile_nt"] = tuple(t)
    else:
        zero[term] = 1.0
    return KernelCosts(**zero)


def features(levels, hq: int, hkv: int):
    """The cost model's count of every term for these levels."""
    return np.array([plan_cost(CostModel(hq, hkv, PAGE, _unit(t)), levels, PAGE)[0] for t in TERMS])


def costs_of(coef) -> KernelCosts:
    c = [round(float(x), 6) for x in coef]
    return KernelCosts(tile_nt=tuple(c[1:5]), seg=c[5], slot=c[6], tail=c[7], fixed=round(float(coef[0]), 3),
                       tile_w128=c[8], tile_w256=c[9], tile_sib=c[10])


def sweep():
    """(name, Hq, Hkv, levels, pages, queries) of the fit's configurations."""
    from .workloads import BUILDERS
    out = []

    def add(name, hq, spec):
        levels, pages = levels_of(spec)
        out.append((name, hq, 8, levels, pages, sum(n for n, _ in spec[0])))
    for hq in (32, 64):
        g = hq // 8
        for nq in (1, 2, 4, 6, 8, 12, 16):
            if nq * g > 64 or (nq in (6, 12) and nq * g != 48):    # 6 / 12 queries: three 16-row tiles
                continue
            for tok in (256, 1024, 4096):
                n = max(4, min(512, int(4e6 // (tok * max(nq, 4) * 4))))
                add(f"g{g}: {n} x ({nq}q, {tok})", hq, [[(nq, tok)] * n])
        for nq in (1, 2, 4):
            for tok in (16, 48, 64):
                add(f"g{g}: 512 x ({nq}q, {tok}) tail", hq, [[(nq, tok)] * 512])
        # groups of two and four 64-row query tiles (the siblings read their K/V from L2)
        for nq in (128 // g, 256 // g):
            for tok in (256, 1024, 4096):
                n = max(4, min(512, int(4e6 // (tok * nq * 4))))
                add(f"g{g}: {n} x ({nq}q, {tok})", hq, [[(nq, tok)] * n])
    for n, suf in ((64, 16), (64, 128), (128, 32)):
        add(f"g4: 8 x (16q, 1024) + {n} x (1q, {suf})", 32, [[(16, 1024)] * 8, [(1, suf)] * 128])
    add("g4: 8 x (16q, 1024) + 128 x (1q, 16) + 128 x (1q, 16)", 32,
        [[(16, 1024)] * 8, [(1, 16)] * 128, [(1, 16)] * 128])
    add("g4: 32 x (4q, 512) + 128 x (1q, 200)", 32, [[(4, 512)] * 32, [(1, 200)] * 128])
    # extra passes without tail chunks: queries split over long groups on two or three levels
    add("g4: 16 x (8q, 1024) + 128 x (1q, 256)", 32, [[(8, 1024)] * 16, [(1, 256)] * 128])
    add("g4: 8 x (16q, 512) + 32 x (4q, 512)", 32, [[(16, 512)] * 8, [(4, 512)] * 32])
    add("g4: 4 x (32q, 1024) + 16 x (8q, 256) + 128 x (1q, 192)", 32,
        [[(32, 1024)] * 4, [(8, 256)] * 16, [(1, 192)] * 128])
    add("g8: 16 x (8q, 512) + 128 x (1q, 512)", 64, [[(8, 512)] * 16, [(1, 512)] * 128])
    # wide segments: groups of 128 / 256+ rows over enough tiles
    add("g8: 2 x (32q, 32768) wide 256", 64, [[(32, 32768)] * 2])
    add("g8: 2 x (24q, 45056) wide 128", 64, [[(24, 45056)] * 2])
    add("g4: 2 x (64q, 32768) wide 256", 32, [[(64, 32768)] * 2])
    add("g8: 2 x (64q, 16384) + 128 x (1q, 256)", 64, [[(64, 16384)] * 2, [(1, 256)] * 128])
    # the benchmark shapes (cascade levels)
    for key in ("c2", "c3", "ns", "e2e", "c5"):
        wl = BUILDERS[key]()
        out.append((f"{key} cascade", wl.hq, wl.hkv, list(zip(*wl.levels)), wl.num_pages, wl.num_queries))
    return out


class _Timer:
    """One level set planned over distinct per-layer caches; ``once()`` times
    the layers back to back (HIP events around the loop): microseconds per
    layer."""

    def __init__(self, levels, pages, nq, hq, hkv):
        import math
        import torch
        from .attention import MultiLevelCascadeAttentionWrapper
        dev = torch.device("cuda")
        per_layer = pages * 2 * PAGE * hkv * D * 2
        self.L = max(4, min(32, math.ceil((1 << 30) / max(per_layer, 1))))
        self.kv = [torch.randn((pages, 2, PAGE, hkv, D), device=dev, dtype=torch.bfloat16) * 0.1
                   for _ in range(self.L)]
        self.q = torch.randn((nq, hq, D), device=dev, dtype=torch.bfloat16) * 0.1
        self.ws = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        self.w = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
        self.w.plan([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
                    hq, hkv, D, PAGE, q_data_type=torch.bfloat16)
        self.out = torch.empty_like(self.q)
        self.ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        for _ in range(3):
            self._layers()
        torch.cuda.synchronize()

    def _layers(self):
        for l in range(self.L):
            self.w.run(self.q, self.kv[l], out=self.out)

    def once(self) -> float:
        import torch
        self.ev[0].record()
        self._layers()
        self.ev[1].record()
        torch.cuda.synchronize()
        return self.ev[0].elapsed_time(self.ev[1]) * 1e3 / self.L


def time_levels(levels, pages, nq, hq, hkv, reps=10):
    """Median microseconds per layer of the cascade wrapper on these levels,
    launches back to back over distinct per-layer caches."""
    import torch
    t = _Timer(levels, pages, nq, hq, hkv)
    us = statistics.median(t.once() for _ in range(reps))
    del t
    torch.cuda.empty_cache()
    return us


def fit(out_path=None):
    from scipy.optimize import nnls
    rows, ys, names = [], [], []
    for name, hq, hkv, levels, pages, nq in sweep():
        us = time_levels(levels, pages, nq, hq, hkv)
        rows.append(features(levels, hq, hkv))
        ys.append(us)
        names.append(name)
        print(f"{name:56s} {us:9.2f} us", flush=True)
    A, y = np.array(rows), np.array(ys)
    w = 1.0 / y                                  # relative error
    coef, _ = nnls(A * w[:, None], y * w)
    costs = costs_of(coef)
    pred = A @ coef
    print(costs)
    res = []
    for n, yy, p in zip(names, y, pred):
        res.append({"config": n, "us": round(float(yy), 2), "model_us": round(float(p), 2)})
        print(f"  {n:56s} measured {yy:9.2f}  model {p:9.2f}  ({100 * (p - yy) / yy:+.0f}%)")
    if out_path:
        with open(out_path, "w") as f:
            json.dump({"costs": {k.name: getattr(costs, k.name) for k in fields(costs)}, "fit": res}, f, indent=1)
    return costs


def table(costs: KernelCosts = MI355X, out_path=None, reps=15):
    """Every option at every benchmark shape: measured and modelled us per
    layer, and the picker's choice.  Options that lay out the same levels are
    timed once (``same_as`` names the first); the distinct plans of a shape
    are timed in interleaved rounds, so that clock drift between them cancels."""
    import torch
    from .workloads import BUILDERS
    rows = []
    for key in ("c2", "c3", "ns", "e2e", "c5"):
        wl = BUILDERS[key]()
        picker = StrategyPicker(wl.hq, wl.hkv, wl.page, costs)
        segs, paths = wl.segment_tree()
        chosen = picker.choose_segments(segs, paths).kind
        opts = {"cascade": list(zip(*wl.levels))}
        for kind in ("flat", "split", "tree", "fasttree"):
            opts[kind] = wl.decomposition(kind, costs)
        canon = {k: tuple(tuple(tuple(int(x) for x in a) for a in lv) for lv in v) for k, v in opts.items()}
        first = {}
        for k in opts:
            first.setdefault(canon[k], k)
        distinct = [k for k in opts if first[canon[k]] == k]
        timers = {k: _Timer(opts[k], wl.num_pages, wl.num_queries, wl.hq, wl.hkv) for k in distinct if k != "flat"}
        samples = {k: [] for k in timers}
        for _ in range(reps):
            for k, t in timers.items():
                samples[k].append(t.once())
        del timers
        torch.cuda.empty_cache()
        flat_us = time_levels(opts["flat"], wl.num_pages, wl.num_queries, wl.hq, wl.hkv, reps=5)
        for kind in opts:
            src = first[canon[kind]]
            us = flat_us if src == "flat" else statistics.median(samples[src])
            model = plan_cost(picker.model, opts[kind], wl.page)[0]
            rows.append({"shape": key, "option": kind, "us": round(us, 2), "model_us": round(model, 2),
                         "picked": kind == chosen, "same_as": src if src != kind else None})
            print(json.dumps(rows[-1]), flush=True)
    if out_path:
        with open(out_path, "w") as f:
            json.dump(rows, f, indent=1)
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None)
    ap.add_argument("--table", action="store_true", help="time and model every option at the benchmark shapes")
    ap.add_argument("--costs", default=None, help="JSON written by --out: table with these costs")
    args = ap.parse_args(argv)
    if args.table:
        costs = MI355X
        if args.costs:
            with open(args.costs) as f:
                c = json.load(f)["costs"]
            costs = replace(MI355X, **{k: (tuple(v) if isinstance(v, list) else v) for k, v in c.items()})
        table(costs, args.out)
    else:
        fit(args.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
