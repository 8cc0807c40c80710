"""Per-step strategy picker: a cost model of this build's decode attention on MI355X.

The reference decides the shape of tree attention in FastTree's preparation
(src/beam_engine/attention/fasttree/preparation.py:34-88): walking the trie top
down, each child node either absorbs its parent's KV into its own pass
(SplitQ: the child's queries read the parent's tokens again, the parent's pass
loses them) or keeps a separate pass whose result is merged (SplitK), whichever
of the two costs less under a padded-tile model Cmm with alpha 0.6, beta 0.3,
gamma 0.1 fitted to its Triton kernel (metadata.py:12-17).  The reference fixes
the strategy per generator (beam.py:20, 168-206) and has no flat strategy.

Here the same top-down edge decision runs over the trie's segments (the
cascade's groups: unbranched page chains) with costs of this build's kernels:
the persistent streaming kernel prices a group by its 64-token tiles — per
tile, by how many 16-row MFMA tiles the group's queries x GQA heads fill —
and by its segment starts; short groups of few queries go to the tail pass,
priced per 16-token chunk; every extra pass of a query costs one partial slot
and its merge.  ``StrategyPicker.choose`` then compares the whole-step costs
of the flat plan (every edge absorbed), the fully split plan and the greedy
edge decision, and returns the cheapest.  All three attend each query to
exactly the tokens of its path (the flat strategy's result), so the choice
changes the time, not the output.

The constants are microseconds per layer on one MI355X, fitted by
``python -m beam_engine_amd.picker_fit`` from timed plans of the streaming
kernel (least squares over a sweep of group shapes).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

from .beam_state import BeamState

TILE_TOKENS = 64          # tokens per streaming-kernel tile
SEG_ROWS = 64             # rows (queries x GQA heads) per streaming segment
TAIL_TOKENS = 128         # tail pass: groups of at most this many tokens ...
TAIL_QUERIES = 4          # ... and at most this many queries
TAIL_CHUNK = 16
WIDE_MIN_TILES = 8        # groups of more than 64 rows take wide (128 / 256-row) segments from this many tiles ...
WIDE_MIN_TILES64 = 64 * 256   # ... when the group alone has 64 tiles of 64 rows per workgroup of an MI355X


@dataclass(frozen=True)
class KernelCosts:
    """Machine time (us per layer, the whole GPU) of one unit of work."""
    tile_nt: Tuple[float, float, float, float] = (0.005492, 0.006099, 0.005898, 0.006712)
    """one 64-token tile of one KV head, by 16-row MFMA tiles filled (1, 2, 3, 4)"""
    seg: float = 0.007525           # a segment start (Q rows, epilogue) of one KV head
    slot: float = 0.0               # a partial slot of one (query, KV head) and its merge (the fit finds it free)
    tail: float = 0.001363          # a 16-token tail chunk of one (query, KV head)
    fixed: float = 12.914           # both launches, prologue and the merge of a step
    tile_w128: float = 0.008329     # one 64-token tile of a 128-row wide segment, one KV head
    tile_w256: float = 0.011948     # one 64-token tile of a 256-row wide segment, one KV head
    tile_sib: float = 0.004881
    """one 64-token tile of a group's second or later 64-row query tile, one KV head: the planner
    places a group's query tiles of one KV head on one XCD at the same tile range, so their K/V
    comes from the L2 the first tile's reads filled"""


MI355X = KernelCosts()


class CostModel:
    """Cost of attention groups for one head configuration and page size."""

    def __init__(self, num_qo_heads: int, num_kv_heads: int, page_size: int, costs: KernelCosts = MI355X):
        self.hkv = num_kv_heads
        self.g = num_qo_heads // num_kv_heads
        self.tail_ok = page_size % 16 == 0 and self.g <= 16
        self.c = costs
        self._memo: Dict[Tuple[int, int], float] = {}

    def group(self, nq: int, tokens: int) -> float:
        """One group of nq queries over `tokens` tokens, all KV heads."""
        if nq <= 0 or tokens <= 0:
            return 0.0
        key = (nq, tokens)
        v = self._memo.get(key)
        if v is None:
            if len(self._memo) > 1 << 16:
                self._memo.clear()
            v = self._memo[key] = self._group(nq, tokens)
        return v

    def _group(self, nq: int, tokens: int) -> float:
        c = self.c
        if self.tail_ok and tokens <= TAIL_TOKENS and nq <= TAIL_QUERIES:
            return nq * self.hkv * math.ceil(tokens / TAIL_CHUNK) * c.tail
        tiles = math.ceil(tokens / TILE_TOKENS)
        rows = nq * self.g
        cost = 0.0
        if rows > SEG_ROWS and tiles >= WIDE_MIN_TILES and \
                math.ceil(rows / SEG_ROWS) * tiles * self.hkv >= WIDE_MIN_TILES64:
            # the planner's wide segments: 256 rows when the group has that many, else 128
            wr, coef = (256, c.tile_w256) if rows >= 256 else (128, c.tile_w128)
            while rows > 0:
                rows -= min(rows, wr)
                cost += tiles * coef + c.seg
            return cost * self.hkv
        first = True
        while rows > 0:
            r = min(rows, SEG_ROWS)
            cost += tiles * (c.tile_nt[min(4, math.ceil(r / 16)) - 1] if first else c.tile_sib) + c.seg
            rows -= r
            first = False
        return cost * self.hkv

    def slots(self, nq: int) -> float:
        return nq * self.hkv * self.c.slot

    def absorb(self, nq_cur: int, nq_child: int, len_parent: int, len_child: int) -> bool:
        """Edge decision (preparation.py:80-85 with this model): True when the
        child should read the parent's tokens in its own pass."""
        split = self.group(nq_cur, len_parent) + self.group(nq_child, len_child) + self.slots(nq_child)
        absorb = self.group(nq_cur - nq_child, len_parent) + self.group(nq_child, len_child + len_parent)
        return absorb < split


class FastTreeCostModel:
    """The reference's own edge model (attention/fasttree/preparation.py:34-57,
    constants of metadata.py:12-38): padded-tile work ``Cmm(nQ, nK) = alpha *
    padQ * g * nK + beta * padK * nQ * g`` with query tiles (64 / g, 16 / g) and
    KV tiles (32, 32) -- the second tile pair when the node has at most 16 / g
    queries -- and a merge when SplitK (separate passes plus gamma per merged
    query) costs more than SplitQ (the child re-reads the parent's KV).  Used
    by ``StrategyPicker(costs="fasttree")`` to decide the tree's edges exactly
    as the reference's FastTree preparation would, on this build's kernels."""

    def __init__(self, num_qo_heads: int, num_kv_heads: int, alpha: float = 0.6, beta: float = 0.3,
                 gamma: float = 0.1):
        self.g = num_qo_heads // num_kv_heads
        self.alpha, self.beta, self.gamma = alpha, beta, gamma
        self.q_tiles = (64 // self.g, 16 // self.g)
        self.kv_tiles = (32, 32)

    def cmm(self, nq: int, nk: int) -> float:
        ph = 0 if nq > self.q_tiles[1] else 1
        tq, tk = self.q_tiles[ph], self.kv_tiles[ph]
        pad_q = tq - ((nq - 1) % tq + 1)
        pad_k = max(0, tk - nk)
        return self.alpha * pad_q * self.g * nk + self.beta * pad_k * nq * self.g

    def absorb(self, nq_cur: int, nq_child: int, len_parent: int, len_child: int) -> bool:
        split_k = self.cmm(nq_cur, len_parent) + self.cmm(nq_child, len_child) + self.gamma * nq_child
        split_q = self.cmm(nq_cur - nq_child, len_parent) + self.cmm(nq_child, len_child + len_parent)
        return split_k > split_q


@dataclass
class Plan:
    kind: str                       # "flat", "split" or "tree"
    levels: List[tuple]             # [(qo_indptr, kv_indptr, kv_indices, last_page_len)] per level
    cost: float
    costs: Dict[str, float] = field(default_factory=dict)   # every option's modelled cost


def decomposition_cost(model: CostModel, segs, paths, absorbed, teff) -> float:
    """Modelled cost of one decomposition of a segment tree: each segment's
    pass over its effective tokens for the candidates it serves, plus a slot
    for every pass of a candidate beyond its first."""
    total = model.c.fixed
    served = [len(s[3]) for s in segs]
    for k in absorbed:
        served[segs[k][2]] -= len(segs[k][3])
    for k, s in enumerate(segs):
        total += model.group(served[k], teff[k])
    extra = 0
    for p in paths:
        passes = sum(1 for j, k in enumerate(p) if teff[k] > 0 and not (j + 1 < len(p) and p[j + 1] in absorbed))
        extra += max(0, passes - 1)
    return total + model.slots(extra)


def plan_cost(model: CostModel, levels: List[tuple], page_size: int) -> Tuple[float, int]:
    """Modelled cost of level arrays (any strategy): their groups, plus a slot
    for every query pass beyond the first.  Returns (cost, groups)."""
    total = model.c.fixed
    passes: Dict[int, int] = {}
    groups = 0
    for qo, kvp, _, lpl in levels:
        for j in range(len(qo) - 1):
            npg = kvp[j + 1] - kvp[j]
            n = 0 if npg == 0 else (npg - 1) * page_size + lpl[j]
            if n <= 0 or qo[j + 1] <= qo[j]:
                continue
            groups += 1
            total += model.group(qo[j + 1] - qo[j], n)
            for q in range(qo[j], qo[j + 1]):
                passes[q] = passes.get(q, 0) + 1
    total += sum(model.slots(1) * (p - 1) for p in passes.values() if p > 1)
    return total, groups


class StrategyPicker:
    """Chooses, per decode step, how the exact path attention of every
    candidate is decomposed: flat (every edge absorbed: one pass per
    candidate over its path), split (no edge absorbed: one pass per trie
    segment, merged), or tree (each edge by ``CostModel.absorb``).  The
    options are costed on the segment tree; only the chosen one is laid out
    as level arrays."""

    def __init__(self, num_qo_heads: int, num_kv_heads: int, page_size: int, costs=MI355X,
                 candidates=("flat", "split", "tree")):
        """``costs``: ``KernelCosts`` (this build's fitted MI355X costs price
        every option and decide the tree's edges) or ``"fasttree"`` (the tree's
        edges decided by the reference's FastTree model, ``FastTreeCostModel``;
        the options are still priced with the MI355X costs)."""
        self.edges = None
        if isinstance(costs, str):
            if costs != "fasttree":
                raise ValueError(f"unknown cost model {costs!r}")
            self.edges = FastTreeCostModel(num_qo_heads, num_kv_heads)
            costs = MI355X
        self.model = CostModel(num_qo_heads, num_kv_heads, page_size, costs)
        self.page_size = page_size
        self.candidates = tuple(candidates)
        self.last: Optional[Plan] = None
        self.history: List[str] = []

    def tree_model(self):
        """These costs and edge decisions as the native planner's model
        (``be_tree_model``: ``be_trie_levels`` / ``be_trie_plan_kind`` decide
        the same edges and price the same options)."""
        from . import _lib
        c = self.model.c
        m = _lib.BeTreeModel()
        for i, v in enumerate(c.tile_nt):
            m.tile_nt[i] = v
        m.seg, m.slot, m.tail, m.fixed = c.seg, c.slot, c.tail, c.fixed
        m.tile_w128, m.tile_w256, m.tile_sib = c.tile_w128, c.tile_w256, c.tile_sib
        ft = self.edges if self.edges is not None else FastTreeCostModel(self.model.g * self.model.hkv, self.model.hkv)
        m.alpha, m.beta, m.gamma = ft.alpha, ft.beta, ft.gamma
        m.num_qo_heads, m.num_kv_heads = self.model.g * self.model.hkv, self.model.hkv
        m.edge_model = _lib.BE_EDGES_FASTTREE if self.edges is not None else _lib.BE_EDGES_FITTED
        return m

    def options(self, segs, paths):
        """Modelled cost and absorbed edge set of every candidate option
        (flat, split, tree) of a segment tree (``BeamState.segment_tree``)."""
        m = self.model
        out = {}
        for kind in self.candidates:
            if kind == "flat":              # every edge absorbed: one pass per candidate over its path
                absorbed = set(k for k, sg in enumerate(segs) if sg[2] >= 0)
                cum = [0] * len(segs)
                for k, sg in enumerate(segs):
                    cum[k] = sg[1] + (cum[sg[2]] if sg[2] >= 0 else 0)
                cost = m.c.fixed + sum(m.group(1, cum[p[-1]]) for p in paths)
            elif kind == "split":           # no edge absorbed: one pass per segment
                absorbed = set()
                cost = decomposition_cost(m, segs, paths, absorbed, [sg[1] for sg in segs])
            else:
                absorbed, teff = BeamState.absorb_edges(segs, (self.edges or m).absorb)
                cost = decomposition_cost(m, segs, paths, absorbed, teff)
            out[kind] = (cost, absorbed)
        return out

    def choose_segments(self, segs, paths) -> Plan:
        """``choose`` on a segment tree given directly."""
        from .beam_state import decomposition_levels
        opts = self.options(segs, paths)
        kind = min(opts, key=lambda k: opts[k][0])
        plan = Plan(kind, decomposition_levels(segs, paths, opts[kind][1], self.page_size), opts[kind][0],
                    {k: v[0] for k, v in opts.items()})
        self.last = plan
        self.history.append(kind)
        return plan

    def costs(self, state: BeamState, include_self: bool = False) -> Dict[str, float]:
        segs, paths = state.segment_tree(include_self)
        return {k: v[0] for k, v in self.options(segs, paths).items()}

    def choose(self, state: BeamState, include_self: bool = False) -> Plan:
        segs, paths = state.segment_tree(include_self)
        return self.choose_segments(segs, paths)
