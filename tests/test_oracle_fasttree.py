"""Pins the FastTree edge-decision restatement (oracle/fasttree.py,
preparation.py:34-88) with hand-evaluated values, and checks the product's
``FastTreeCostModel`` / ``BeamState.absorb_edges`` against it.

Hand arithmetic below uses g = 32 / 8 = 4, so TSQ = (16, 4), TSK = (32, 32):
a node with more than 4 queries uses the first tile pair."""

import random

import pytest

from beam_engine_amd.beam_state import BeamState
from beam_engine_amd.picker import FastTreeCostModel
from oracle import fasttree as ft

G = 4


def close(a, b):
    return abs(a - b) < 1e-9


def test_padding_hand_values():
    assert ft.cpad_q(16, 5) == 11          # 16 - ((4 % 16) + 1)
    assert ft.cpad_q(16, 16) == 0
    assert ft.cpad_q(16, 17) == 15         # 16 - ((16 % 16) + 1)
    assert ft.cpad_q(4, 0) == 0            # Python modulo: (-1) % 4 = 3 -> 4 - 4
    assert ft.cpad_k(32, 10) == 22
    assert ft.cpad_k(32, 40) == 0


def test_cmm_hand_values():
    # phase 0 (8 > 4): 0.6 * cpadQ(16, 8) * 4 * 100 + 0.3 * cpadK(32, 100) * 8 * 4 = 0.6 * 8 * 400 + 0
    assert close(ft.cmm(8, 100, G), 1920.0)
    # phase 1 (2 <= 4): 0.6 * cpadQ(4, 2) * 4 * 10 + 0.3 * cpadK(32, 10) * 2 * 4 = 48 + 52.8
    assert close(ft.cmm(2, 10, G), 100.8)
    # 0.6 * 2 * 4 * 8 + 0.3 * 24 * 2 * 4 = 38.4 + 57.6; alpha and beta exchanged would give 134.4
    assert close(ft.cmm(2, 8, G), 96.0)
    assert close(ft.cmm(3, 8, G), 105.6)    # 0.6 * 1 * 32 + 0.3 * 24 * 12
    assert close(ft.cmm(1, 16, G), 134.4)   # 0.6 * 3 * 64 + 0.3 * 16 * 4
    assert close(ft.cmm(0, 8, G), 0.0)


def test_split_costs_hand_values():
    # SplitK(16, 1, lenl 32, lenv 1024) = Cmm(16, 1024) + Cmm(1, 32) + 0.1 = 0 + 0.6 * 3 * 4 * 32 + 0.1;
    # exchanging the two lengths would give Cmm(16, 32) + Cmm(1, 1024) + 0.1 = 7372.9
    assert close(ft.split_k_cost(16, 1, 32, 1024, G), 230.5)
    # SplitQ(16, 1, lenv 1024, lenl 32) = Cmm(15, 1024) + Cmm(1, 1056) = 2457.6 + 7603.2
    assert close(ft.split_q_cost(16, 1, 1024, 32, G), 10060.8)
    assert not ft.merge_into_parent(16, 1, 1024, 32, G)
    # 5 queries over 8 tokens, a 4-query child over 8 more: SplitK = 355.2 + 115.2 + 0.4 > SplitQ = 86.4 + 76.8
    assert close(ft.split_k_cost(5, 4, 8, 8, G), 470.8)
    assert close(ft.split_q_cost(5, 4, 8, 8, G), 163.2)
    assert ft.merge_into_parent(5, 4, 8, 8, G)


def test_edge_assignments_sibling_count():
    """Root with 3 queries over 8 tokens, children of 2 and 1 queries over 8.
    Child 1: SplitK = Cmm(3,8) + Cmm(2,8) + 0.2 = 105.6 + 96 + 0.2 = 201.8 >
    SplitQ = Cmm(1,8) + Cmm(2,16) = 86.4 + 115.2 = 201.6 -> merge, the root keeps 1
    query.  Child 2: SplitK = 86.4 + 86.4 + 0.1 = 172.9 > SplitQ = Cmm(0,8) +
    Cmm(1,16) = 134.4 -> merge.  Had the root kept 3 queries: SplitK = 105.6 +
    86.4 + 0.1 = 192.1 < SplitQ = 96 + 134.4 = 230.4 -> split."""
    a = ft.edge_assignments([-1, 0, 0], [8, 8, 8], [[0, 1, 2], [0, 1], [2]], 32, 8)
    assert a == [0, 1, 1]


def test_edge_assignments_extended_length():
    """Chain 0 -> 1 -> 2 of 3, 3, 2 queries over 8 tokens each.  Edge 0-1:
    SplitK = 105.6 + 105.6 + 0.3 = 211.5 > SplitQ = Cmm(0,8) + Cmm(3,16) = 96 ->
    merge, node 1 now spans 16 tokens.  Edge 1-2: SplitK = Cmm(3,16) + Cmm(2,8)
    + 0.2 = 192.2 < SplitQ = Cmm(1,16) + Cmm(2,24) = 134.4 + 76.8 = 211.2 ->
    split.  With node 1's original 8 tokens it would merge (201.8 > 201.6)."""
    a = ft.edge_assignments([-1, 0, 1], [8, 8, 8], [[0, 1, 2], [0, 1, 2], [0, 1]], 32, 8)
    assert a == [0, 1, 0]


def test_edge_assignments_root_and_leaves_unmerged():
    a = ft.edge_assignments([-1], [100], [[0]], 32, 8)
    assert a == [0]
    # a long shared root with one-query leaves: never worth re-reading (SplitQ >> SplitK)
    a = ft.edge_assignments([-1, 0, 0, 0], [4096, 4128, 4128, 4128], [[0, 1, 2], [0], [1], [2]], 32, 8)
    assert a == [0, 0, 0, 0]


@pytest.mark.parametrize("g", [1, 2, 4, 8])
def test_product_model_equals_oracle(g):
    m = FastTreeCostModel(8 * g, 8)
    rng = random.Random(g)
    for _ in range(3000):
        nq = rng.randint(1, 70)
        nc = rng.randint(1, nq)
        lp, lc = rng.choice([1, 7, 16, 31, 32, 33, 100, 1024]), rng.choice([1, 5, 16, 32, 64, 129])
        assert m.absorb(nq, nc, lp, lc) == ft.merge_into_parent(nq, nc, lp, lc, g)
        assert abs(m.cmm(nq, lp) - ft.cmm(nq, lp, g)) < 1e-9


def random_tree(rng, n):
    """BFS-numbered tree with per-node query sets (a node's queries are the
    union of its children's, leaves own fresh ones) and node lengths."""
    parents = [-1]
    for i in range(1, n):
        parents.append(rng.randrange(i))
    kids = [[] for _ in range(n)]
    for i in range(1, n):
        kids[parents[i]].append(i)
    # renumber in BFS order so that children follow index order as in the reference
    order, q = [], [0]
    while q:
        x = q.pop(0)
        order.append(x)
        q.extend(kids[x])
    new = {o: i for i, o in enumerate(order)}
    par = [-1 if parents[o] < 0 else new[parents[o]] for o in order]
    ch = [[] for _ in range(n)]
    for i in range(1, n):
        ch[par[i]].append(i)
    reqs = [None] * n
    nxt = 0
    for i in reversed(range(n)):
        if not ch[i]:
            k = rng.randint(1, 4)
            reqs[i] = list(range(nxt, nxt + k))
            nxt += k
        else:
            reqs[i] = sorted(x for c in ch[i] for x in reqs[c])
    lens = [rng.choice([1, 8, 16, 32, 64, 200]) for _ in range(n)]
    return par, ch, reqs, lens


def test_product_absorb_edges_equals_oracle_bfs():
    """BeamState.absorb_edges with the reference model makes the oracle's BFS
    decisions (sibling count and length extension included) on random trees
    given as segments (parents before children, children in index order)."""
    rng = random.Random(5)
    for _ in range(300):
        n = rng.randint(1, 12)
        par, ch, reqs, lens = random_tree(rng, n)
        segs = [[None, lens[i], par[i], reqs[i], ch[i]] for i in range(n)]
        absorbed, teff = BeamState.absorb_edges(segs, FastTreeCostModel(32, 8).absorb)
        want = ft.edge_assignments(par, lens, reqs, 32, 8)
        assert [1 if i in absorbed else 0 for i in range(n)] == want
