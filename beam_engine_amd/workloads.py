"""Synthetic decode-attention workloads at the benchmark configurations.

Each builder returns a ``Workload``: cascade levels (per-level qo_indptr,
kv_indptr, kv_indices, last_page_len), the flat arrays over the same pages
(one group per query = its root-to-leaf path), the page count and the head
shape.  Pages are numbered in allocation order; every non-last page of a
group is full.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List

import numpy as np


@dataclass
class Workload:
    name: str
    hq: int
    hkv: int
    d: int
    page: int
    num_queries: int
    num_pages: int
    levels: tuple                      # (qo_arr, kvp_arr, kvi_arr, lpl_arr)
    flat: tuple                        # (kv_indptr, kv_indices, last_page_len)
    note: str = ""
    tokens_per_query: List[int] = field(default_factory=list)

    def segment_tree(self):
        """(segs, paths) as ``BeamState.segment_tree`` gives them, read off
        the cascade levels (each group is one segment, its parent the group
        one level up holding its queries; every query has a group on every
        level here)."""
        qo_arr, kvp_arr, kvi_arr, lpl_arr = self.levels
        segs, paths = [], [[] for _ in range(self.num_queries)]
        prev_of = [-1] * self.num_queries
        for qo, kvp, kvi, lpl in zip(qo_arr, kvp_arr, kvi_arr, lpl_arr):
            for j in range(len(qo) - 1):
                pages = list(kvi[kvp[j]: kvp[j + 1]])
                qs = list(range(qo[j], qo[j + 1]))
                parent = prev_of[qs[0]]
                if any(prev_of[q] != parent for q in qs):
                    raise ValueError("a group's queries have different parents")
                k = len(segs)
                segs.append([pages, (len(pages) - 1) * self.page + int(lpl[j]), parent, qs, []])
                if parent >= 0:
                    segs[parent][4].append(k)
                for q in qs:
                    paths[q].append(k)
                    prev_of[q] = k
        return segs, paths

    def decomposition(self, kind: str, costs=None):
        """Level arrays of one exact path decomposition of the workload:
        "flat", "split", "tree" (the fitted MI355X edge model, or ``costs``),
        "fasttree" (FastTree's edge model) or "auto" (the picker's choice)."""
        from .beam_state import BeamState, decomposition_levels
        from .picker import MI355X, StrategyPicker
        segs, paths = self.segment_tree()
        picker = StrategyPicker(self.hq, self.hkv, self.page,
                                "fasttree" if kind == "fasttree" else (costs if costs is not None else MI355X))
        if kind == "auto":
            return picker.choose_segments(segs, paths).levels
        if kind == "flat":
            absorbed = set(k for k, sg in enumerate(segs) if sg[2] >= 0)
        elif kind == "split":
            absorbed = set()
        elif kind in ("tree", "fasttree"):
            absorbed, _ = BeamState.absorb_edges(segs, (picker.edges or picker.model).absorb)
        else:
            raise ValueError(f"unknown decomposition {kind!r}")
        return decomposition_levels(segs, paths, absorbed, self.page)


class _Pages:
    def __init__(self):
        self.next = 0

    def take(self, tokens: int, page: int):
        n = max(1, -(-tokens // page))
        out = list(range(self.next, self.next + n))
        self.next += n
        return out, tokens - (n - 1) * page


def _flat_from_paths(paths):
    kvp, kvi, lpl = [0], [], []
    for pages, last in paths:
        kvi.extend(pages)
        kvp.append(len(kvi))
        lpl.append(last)
    return kvp, kvi, lpl


def shared_prefix(name, n_req, beams, prefix, suffixes, hq, hkv, d, page=16, note=""):
    """Two-level cascade: a shared prefix per request, a private suffix per beam."""
    alloc = _Pages()
    lv0 = ([0], [0], [], [])
    lv1 = ([0], [0], [], [])
    paths = []
    for r in range(n_req):
        pp, plast = alloc.take(prefix, page)
        lv0[2].extend(pp)
        lv0[1].append(len(lv0[2]))
        lv0[3].append(plast)
        lv0[0].append(lv0[0][-1] + beams)
        for b in range(beams):
            s = int(suffixes[r * beams + b])
            sp, slast = alloc.take(s, page)
            lv1[2].extend(sp)
            lv1[1].append(len(lv1[2]))
            lv1[3].append(slast)
            lv1[0].append(lv1[0][-1] + 1)
            assert plast == page, "prefix must fill its last page for a flat path"
            paths.append((pp + sp, slast))
    levels = tuple([lv0[i], lv1[i]] for i in range(4))
    n = n_req * beams
    return Workload(name, hq, hkv, d, page, n, alloc.next, levels, _flat_from_paths(paths), note,
                    [prefix + int(s) for s in suffixes])


def config2():
    """Kernel-level cascade shape: 4 requests x beam 8, Llama-3-8B GQA 32/8, D 128, prefix 2048, suffix 128."""
    return shared_prefix("c2", 4, 8, 2048, [128] * 32, 32, 8, 128,
                         note="4 req x beam 8, 32/8 heads, D128, bf16, page 16, prefix 2048, suffix 128")


def north_star():
    """Llama-3-8B GQA shape at beam 16 with a 4k shared prefix (the north-star
    target shape): 8 requests x beam 16, prefix 4096, suffix 128 per beam."""
    return shared_prefix("ns", 8, 16, 4096, [128] * 128, 32, 8, 128,
                         note="8 req x beam 16, 32/8 heads, D128, bf16, page 16, prefix 4096, suffix 128")


def config5(seed: int = 5):
    """Long-context stress shape: 70B layer shape 64/8, 2 requests x beam 64, prefix 32768,
    suffix ~ U[1, 512] per beam from ``seed``."""
    rng = np.random.default_rng(seed)
    suf = rng.integers(1, 513, size=128)
    return shared_prefix("c5", 2, 64, 32768, suf.tolist(), 64, 8, 128,
                         note=f"2 req x beam 64, 64/8 heads, D128, bf16, prefix 32768, suffix U[1,512] seed {seed}")


def config3():
    """Multi-level tree, beam 32, root 4096, fanout 2/4/4 with node lengths
    256/128/64 and a 32-token leaf suffix (4 levels; the last chain and the
    suffix form one level)."""
    page = 16
    alloc = _Pages()
    root, _ = alloc.take(4096, page)
    l1 = [alloc.take(256, page)[0] for _ in range(2)]
    l2 = [alloc.take(128, page)[0] for _ in range(8)]
    l3 = [alloc.take(64, page)[0] + alloc.take(32, page)[0] for _ in range(32)]
    levels = ([[0, 32], [0, 16, 32], list(range(0, 33, 4)), list(range(33))],
              [[0, len(root)], [0, 16, 32], list(range(0, 65, 8)), list(range(0, 193, 6))],
              [root, sum(l1, []), sum(l2, []), sum(l3, [])],
              [[16], [16, 16], [16] * 8, [16] * 32])
    paths = []
    for leaf in range(32):
        p = root + l1[leaf // 16] + l2[leaf // 4] + l3[leaf]
        paths.append((p, 16))
    return Workload("c3", 32, 8, 128, page, 32, alloc.next, levels, _flat_from_paths(paths),
                    "tree: beam 32, root 4096, fanout 2/4/4 x 256/128/64, leaf suffix 32, 32/8 heads, D128, bf16",
                    [4096 + 256 + 128 + 96] * 32)


def e2e_step():
    """The decode attention of one config-4 step (8 requests x beam 16, 32/8
    heads, D 128, bf16, page 16) at the trie's typical mid-run structure:
    each request's 16 beams share a 1136-token prefix (the 1024-token prompt
    and the generated tokens all beams agree on), then branch into groups of
    1, 1, 2, 3, 1 and 8 beams over one 16-token page each, and every beam ends
    in a private page holding 8 tokens (three cascade levels)."""
    page = 16
    alloc = _Pages()
    split = [1, 1, 2, 3, 1, 8]
    lv = [([0], [0], [], []) for _ in range(3)]
    paths = []

    def add(level, pages, last, nq):
        qo, kvp, kvi, lpl = lv[level]
        kvi.extend(pages)
        kvp.append(len(kvi))
        lpl.append(last)
        qo.append(qo[-1] + nq)
    for r in range(8):
        pre, last0 = alloc.take(1136, page)
        add(0, pre, last0, 16)
        for nb in split:
            mid, last1 = alloc.take(16, page)
            add(1, mid, last1, nb)
            for _ in range(nb):
                leaf, last2 = alloc.take(8, page)
                add(2, leaf, last2, 1)
                paths.append((pre + mid + leaf, last2))
    levels = tuple([l[i] for l in lv] for i in range(4))
    return Workload("e2e", 32, 8, 128, page, 128, alloc.next, levels, _flat_from_paths(paths),
                    "config-4 step: 8 req x beam 16, 32/8 heads, D128, bf16, prefix 1136, branch pages of 16, "
                    "leaf pages of 8", [1136 + 16 + 8] * 128)


def config1():
    """CPU-path shape: 1 request x beam 4, prefix 512, suffix 32, 8/8 heads, D 64, fp32, page 16."""
    return shared_prefix("c1", 1, 4, 512, [32] * 4, 8, 8, 64,
                         note="1 req x beam 4, 8/8 heads, D64, fp32, page 16, prefix 512, suffix 32")


BUILDERS = {"c1": config1, "c2": config2, "c3": config3, "c5": config5, "ns": north_star, "e2e": e2e_step}
