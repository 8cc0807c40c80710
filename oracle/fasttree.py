"""CPU restatement of FastTree's SplitQ / SplitK edge decisions (test infrastructure).

Follows src/beam_engine/attention/fasttree/preparation.py:34-88 and the
defaults of metadata.py:12-38 (alpha 0.6, beta 0.3, gamma 0.1,
TSQ = (64 // g, 16 // g), TSK = (32, 32), g = num_qo_heads // num_kv_heads).

Pinned by hand-evaluated values of every cost function and of the edge
decisions of small trees (tests/test_oracle_fasttree.py), including a tree
whose second edge decision flips when an earlier sibling's merge is not
subtracted from the parent's query count, and planted mistakes (swapped
lengths, alpha / beta exchanged) that those values reject.
"""

from __future__ import annotations

from collections import deque
from typing import List, Sequence

ALPHA, BETA, GAMMA = 0.6, 0.3, 0.1
TSK = (32, 32)


def tile_sizes(g: int):
    """TSQs of metadata.py:33-35 for GQA group g."""
    return (64 // g, 16 // g)


def cpad_q(ts: int, n: int) -> int:
    """Query-tile padding, preparation.py:41-42 (Python's modulo for n = 0)."""
    return ts - ((n - 1) % ts + 1)


def cpad_k(ts: int, n: int) -> int:
    """KV-tile padding, preparation.py:44-45."""
    return max(0, ts - n)


def cmm(nq: int, nk: int, g: int, alpha=ALPHA, beta=BETA, tsq=None, tsk=TSK) -> float:
    """Padded-work cost of one node, preparation.py:47-51: phase 0 when the
    node has more queries than the second phase's query tile."""
    if tsq is None:
        tsq = tile_sizes(g)
    phase = 0 if nq > tsq[1] else 1
    return alpha * cpad_q(tsq[phase], nq) * g * nk + beta * cpad_k(tsk[phase], nk) * nq * g


def split_q_cost(nq_cur: int, nq_child: int, len_parent: int, len_child: int, g: int, **kw) -> float:
    """SplitQCost(nQcurr, nQl, lenv, lenl), preparation.py:53-54: the child's
    queries read the parent's KV in the child's pass."""
    return cmm(nq_cur - nq_child, len_parent, g, **kw) + cmm(nq_child, len_child + len_parent, g, **kw)


def split_k_cost(nq_cur: int, nq_child: int, len_child: int, len_parent: int, g: int,
                 gamma: float = GAMMA, **kw) -> float:
    """SplitKCost(nQcurr, nQl, lenl, lenv), preparation.py:56-57: separate
    parent and child passes plus the merge of the child's queries."""
    return cmm(nq_cur, len_parent, g, **kw) + cmm(nq_child, len_child, g, **kw) + gamma * nq_child


def merge_into_parent(nq_cur: int, nq_child: int, len_parent: int, len_child: int, g: int) -> bool:
    """Edge decision of preparation.py:80-85: merge (assignment 1) when
    SplitK > SplitQ."""
    return split_k_cost(nq_cur, nq_child, len_child, len_parent, g) > \
        split_q_cost(nq_cur, nq_child, len_parent, len_child, g)


def edge_assignments(parents: Sequence[int], seqlens: Sequence[int], requests: Sequence[Sequence[int]],
                     num_qo_heads: int, num_kv_heads: int) -> List[int]:
    """``node_assignments`` of preparation.py:60-88 for a KVTreeNode list given
    as parallel arrays (kv_tree_node.py:3-19): BFS from node 0; for each child
    in index order, merge into the parent (1) when SplitK > SplitQ with the
    parent's current query count and (possibly already extended) length; a
    merge subtracts the child's queries from the parent's count and extends
    the child's length by the parent's.  ``seqlens`` are used as given: the
    reference passes cumulative lengths here (beam_state.py:480-486)."""
    g = num_qo_heads // num_kv_heads
    n = len(parents)
    edges: List[List[int]] = [[] for _ in range(n)]
    for i in range(n):
        if parents[i] != -1:
            edges[parents[i]].append(i)
    length = list(seqlens)
    assign = [0] * n
    que = deque([0])
    while que:
        node = que.popleft()
        nq_cur = len(requests[node])
        lenv = length[node]
        for child in edges[node]:
            nql = len(requests[child])
            lenl = length[child]
            if split_k_cost(nq_cur, nql, lenl, lenv, g) > split_q_cost(nq_cur, nql, lenv, lenl, g):
                assign[child] = 1
                nq_cur -= nql
                length[child] = lenl + lenv
            que.append(child)
    return assign
