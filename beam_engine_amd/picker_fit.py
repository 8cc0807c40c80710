"""Fits the picker's kernel costs on the GPU at hand.

``python -m beam_engine_amd.picker_fit [--out FILE]`` times the cascade
wrapper (streaming kernel + tail-and-merge kernel, bf16, Hq 32 / Hkv 8,
head_dim 128, page 16) on a sweep of synthetic level sets — long groups of
1..16 queries (one to four 16-row MFMA tiles per KV head), short groups that
take the tail pass, and two-level sets whose queries need partial slots —
each over enough distinct per-layer caches to stream from HBM, and solves a
non-negative least-squares fit of

    us per layer = fixed + sum_nt tile_nt * tiles(nt) + seg * segments
                   + slot * extra passes + tail * tail chunks

(counted as ``picker.CostModel`` counts them).  Prints the fitted
``KernelCosts`` and the per-configuration residuals; ``--out`` writes them as
JSON.
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import sys

import numpy as np

from .picker import SEG_ROWS, TAIL_CHUNK, TAIL_QUERIES, TAIL_TOKENS, TILE_TOKENS, KernelCosts

HQ, HKV, D, PAGE = 32, 8, 128, 16
G = HQ // HKV


def levels_of(spec):
    """spec: list of levels, each a list of (queries, tokens) groups in query
    order; every level covers the same queries.  Returns (levels, pages)."""
    page = 0
    out = []
    for groups in spec:
        qo, kvp, kvi, lpl = [0], [0], [], []
        for nq, tok in groups:
            npg = -(-tok // PAGE)
            kvi.extend(range(page, page + npg))
            page += npg
            kvp.append(len(kvi))
            lpl.append(tok - (npg - 1) * PAGE)
            qo.append(qo[-1] + nq)
        out.append((qo, kvp, kvi, lpl))
    return out, page


def features(spec):
    """[fixed, tiles nt=1..4, segments, extra passes, tail chunks] of a spec."""
    f = np.zeros(8)
    f[0] = 1.0
    nq_total = sum(nq for nq, _ in spec[0])
    passes = np.zeros(nq_total)
    for groups in spec:
        q = 0
        for nq, tok in groups:
            if tok > 0:
                passes[q:q + nq] += 1
                if tok <= TAIL_TOKENS and nq <= TAIL_QUERIES:
                    f[7] += nq * HKV * math.ceil(tok / TAIL_CHUNK)
                else:
                    tiles = math.ceil(tok / TILE_TOKENS)
                    rows = nq * G
                    while rows > 0:
                        r = min(rows, SEG_ROWS)
                        f[min(4, math.ceil(r / 16))] += tiles * HKV
                        f[5] += HKV
                        rows -= r
            q += nq
    f[6] = np.maximum(passes - 1, 0).sum() * HKV
    return f


def sweep():
    specs = []
    for nq in (1, 2, 4, 8, 12, 16):
        for tok in (256, 1024, 4096):
            n = max(4, min(512, int(4e6 // (tok * max(nq, 4) * 4))))
            specs.append((f"{n} x ({nq}q, {tok})", [[(nq, tok)] * n]))
    for nq in (1, 2, 4):
        for tok in (16, 48, 64):
            specs.append((f"512 x ({nq}q, {tok}) tail", [[(nq, tok)] * 512]))
    for n, suf in ((64, 16), (64, 128), (128, 32)):
        specs.append((f"8 x (16q, 1024) + {128} x (1q, {suf})",
                      [[(16, 1024)] * 8, [(1, suf)] * 128]))
    specs.append(("8 x (16q, 1024) + 128 x (1q, 16) + 128 x (1q, 16)",
                  [[(16, 1024)] * 8, [(1, 16)] * 128, [(1, 16)] * 128]))
    specs.append(("32 x (4q, 512) + 128 x (1q, 200)", [[(4, 512)] * 32, [(1, 200)] * 128]))
    return specs


def time_spec(levels, pages, nq, reps=10):
    import torch
    from .attention import MultiLevelCascadeAttentionWrapper
    dev = torch.device("cuda")
    per_layer = pages * 2 * PAGE * HKV * D * 2
    L = max(4, min(32, math.ceil((1 << 30) / max(per_layer, 1))))
    kv = [torch.randn((pages, 2, PAGE, HKV, D), device=dev, dtype=torch.bfloat16) * 0.1 for _ in range(L)]
    q = torch.randn((nq, HQ, D), device=dev, dtype=torch.bfloat16) * 0.1
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    w = MultiLevelCascadeAttentionWrapper(len(levels), ws)
    w.plan([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
           HQ, HKV, D, PAGE, q_data_type=torch.bfloat16)
    out = torch.empty_like(q)
    for _ in range(3):
        for l in range(L):
            w.run(q, kv[l], out=out)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ts = []
    for _ in range(reps):
        ev[0].record()
        for l in range(L):
            w.run(q, kv[l], out=out)
        ev[1].record()
        torch.cuda.synchronize()
        ts.append(ev[0].elapsed_time(ev[1]) * 1e3 / L)
    del kv
    return statistics.median(ts)


def main(argv=None):
    from scipy.optimize import nnls
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None)
    args = ap.parse_args(argv)
    rows, ys, names = [], [], []
    for name, spec in sweep():
        levels, pages = levels_of(spec)
        nq = sum(n for n, _ in spec[0])
        us = time_spec(levels, pages, nq)
        rows.append(features(spec))
        ys.append(us)
        names.append(name)
        print(f"{name:52s} {us:8.2f} us", flush=True)
    A, y = np.array(rows), np.array(ys)
    w = 1.0 / y                                  # relative error
    coef, _ = nnls(A * w[:, None], y * w)
    costs = KernelCosts(tile_nt=tuple(round(float(c), 6) for c in coef[1:5]), seg=round(float(coef[5]), 6),
                        slot=round(float(coef[6]), 6), tail=round(float(coef[7]), 6), fixed=round(float(coef[0]), 3))
    pred = A @ coef
    print(costs)
    res = []
    for n, yy, p in zip(names, y, pred):
        res.append({"config": n, "us": round(float(yy), 2), "model_us": round(float(p), 2)})
        print(f"  {n:52s} measured {yy:8.2f}  model {p:8.2f}  ({100 * (p - yy) / yy:+.0f}%)")
    if args.out:
        with open(args.out, "w") as f:
            json.dump({"costs": costs.__dict__, "fit": res}, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
