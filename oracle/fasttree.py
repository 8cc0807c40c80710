"""CPU restatement of the FastTree SplitQ / SplitK cost model (test infrastructure).

Follows src/beam_engine/attention/fasttree/preparation.py:34-57 and the
defaults of metadata.py:12-38 (alpha 0.6, beta 0.3, gamma 0.1,
TSQ = (64 // g, 16 // g), TSK = (32, 32)).
"""

from __future__ import annotations


def cpad_q(ts: int, n: int) -> int:
    """Query-tile padding, preparation.py:41-42."""
    return ts - ((n - 1) % ts + 1)


def cpad_k(ts: int, n: int) -> int:
    """KV-tile padding, preparation.py:44-45."""
    return max(0, ts - n)


def cmm(nq: int, nk: int, g: int, alpha=0.6, beta=0.3, tsq=None, tsk=(32, 32)) -> float:
    """Padded-work cost of one node, preparation.py:47-51."""
    if tsq is None:
        tsq = (64 // g, 16 // g)
    phase = 0 if nq > tsq[1] else 1
    return alpha * cpad_q(tsq[phase], nq) * g * nk + beta * cpad_k(tsk[phase], nk) * nq * g


def split_q_cost(nq_cur: int, nq_child: int, len_parent: int, len_child: int, g: int, **kw) -> float:
    """Cost of folding the parent's KV into the child's pass, preparation.py:53-54."""
    return cmm(nq_cur - nq_child, len_parent, g, **kw) + cmm(nq_child, len_child + len_parent, g, **kw)


def split_k_cost(nq_cur: int, nq_child: int, len_child: int, len_parent: int, g: int,
                 gamma: float = 0.1, **kw) -> float:
    """Cost of separate parent and child passes plus a merge, preparation.py:56-57."""
    return cmm(nq_cur, len_parent, g, **kw) + cmm(nq_child, len_child, g, **kw) + gamma * nq_child


def merge_into_parent(nq_cur: int, nq_child: int, len_parent: int, len_child: int, g: int) -> bool:
    """Edge decision of preparation.py:80-85: merge when SplitK > SplitQ."""
    return split_k_cost(nq_cur, nq_child, len_child, len_parent, g) > \
        split_q_cost(nq_cur, nq_child, len_parent, len_child, g)
